"""Writes the small golden fixtures under tests/golden/ from the CPU oracle in fp64.

The reference repository ships no golden vectors, so these fixtures are generated from the
oracle restatement (itself pinned by tests/test_oracle.py against brute force and closed
forms).  Inputs are drawn N(0,1), rounded to bf16 and stored as fp32 so that the same
values feed both the bf16 and the fp32 code paths; shapes are ragged on purpose.

Run:  python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import reference as ref  # noqa: E402

BASED_CASES = [
    # name, B, H, N, d, dv, seed, prescale
    ("based_b1h2n67d16dv64", 1, 2, 67, 16, 64, 11, True),
    ("based_b1h1n130d16dv16", 1, 1, 130, 16, 16, 12, True),
    ("based_b1h2n129d4dv8", 1, 2, 129, 4, 8, 13, True),
    ("based_b1h2n67d16dv64_unscaled", 1, 2, 67, 16, 64, 14, False),
]

SLIDING_CASES = [
    # name, B, H, N, d, dv, seed, window
    ("sliding_b1h2n131d64w1", 1, 2, 131, 64, 64, 21, 1),
    ("sliding_b1h2n131d64w17", 1, 2, 131, 64, 64, 22, 17),
    ("sliding_b1h2n131d64w64", 1, 2, 131, 64, 64, 23, 64),
]

FEATURE_CASES = [
    ("phi_d4", 5, 4, 31),
    ("phi_d16", 7, 16, 32),
]


def _bf16_inputs(B, H, N, d, dv, seed, prescale):
    q, k, v = ref.make_inputs(B, H, N, d, dv, torch.bfloat16, seed, prescale)
    return q.float(), k.float(), v.float()


def main():
    for name, B, H, N, d, dv, seed, prescale in BASED_CASES:
        q, k, v = _bf16_inputs(B, H, N, d, dv, seed, prescale)
        y, num, den = ref.based_dense(q, k, v, dtype=torch.float64)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), q=q.numpy(), k=k.numpy(), v=v.numpy(),
                            y=y.numpy(), num=num.numpy(), den=den.numpy(), eps=np.float64(ref.EPS))
    for name, B, H, N, d, dv, seed, w in SLIDING_CASES:
        q, k, v = _bf16_inputs(B, H, N, d, dv, seed, False)
        y = ref.sliding_dense(q, k, v, window_size=w, dtype=torch.float64)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), q=q.numpy(), k=k.numpy(), v=v.numpy(),
                            y=y.numpy(), window=np.int64(w))
    for name, rows, d, seed in FEATURE_CASES:
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(rows, d, generator=g).to(torch.bfloat16).float()
        phi = ref.taylor_feature_map(x.double())
        np.savez_compressed(os.path.join(HERE, name + ".npz"), x=x.numpy(), phi=phi.numpy())
    print("wrote", len(BASED_CASES) + len(SLIDING_CASES) + len(FEATURE_CASES), "fixtures to", HERE)


if __name__ == "__main__":
    main()
