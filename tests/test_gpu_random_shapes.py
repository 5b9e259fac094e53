"""Seeded random shapes through every kernel path against the fp64 oracle: batch, heads, length,
head dims, window, dtype and scale drawn per case (the cases are fixed by the seed, so a failure
names a reproducible shape)."""

import math

import numpy as np
import pytest
import torch

from oracle import reference as ref
from tests.helpers import err, rand_qkv, to_dev

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 2e-2, torch.float32: 1e-4}


def _kernels():
    import kernels
    return kernels


def _cases(kind, n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        B, H = int(rng.integers(1, 4)), int(rng.integers(1, 5))
        N = int(rng.choice([int(rng.integers(1, 80)), int(rng.integers(80, 700))]))
        dtype = torch.bfloat16 if rng.random() < 0.75 else torch.float32
        if kind in ("chunked", "identity"):
            dtype = torch.bfloat16
        if kind == "chunked":
            d, dv = 16, int(rng.choice([8, 16, 24, 32, 40, 64]))
        elif kind == "identity":
            d, dv = int(rng.choice([4, 16, 20, 32, 64])), int(rng.choice([1, 16, 32, 48, 64, 100]))
        else:
            d = int(rng.choice([4, 8, 16, 24, 32, 64, 128]))
            dv = int(rng.choice([1, 8, 16, 32, 48, 64, 96, 128]))
        W = int(rng.choice([1, 7, 64, 65, int(rng.integers(1, 300))]))
        sq = float(rng.choice([0.25, 0.5, 1.0]))
        out.append(pytest.param(B, H, N, d, dv, W, dtype, sq, 1000 * seed + i,
                                id=f"{kind}-B{B}H{H}N{N}d{d}dv{dv}W{W}-{str(dtype)[6:]}-s{sq}"))
    return out


@pytest.mark.parametrize("B,H,N,d,dv,W,dtype,sq,seed", _cases("parallel", 24, 1))
def test_parallel(B, H, N, d, dv, W, dtype, sq, seed):
    K = _kernels()
    q, k, v = rand_qkv(B, H, N, d, dv, seed=seed, dtype=dtype, scale_qk=sq / math.sqrt(math.sqrt(d)))
    y, den = K.based_parallel(*to_dev(q, k, v), out_dtype=torch.float32, return_den=True)
    want, _, want_den = ref.based_dense(q, k, v)
    assert err(y, want) < TOL[dtype]
    assert err(den, want_den) < TOL[dtype]


@pytest.mark.parametrize("B,H,N,d,dv,W,dtype,sq,seed", _cases("chunked", 16, 2))
def test_chunked(B, H, N, d, dv, W, dtype, sq, seed):
    K = _kernels()
    q, k, v = rand_qkv(B, H, N, d, dv, seed=seed, dtype=dtype, scale_qk=sq / 2.0)
    y = K.based_chunked(*to_dev(q, k, v), out_dtype=torch.float32)
    want, _, _ = ref.based_dense(q, k, v)
    assert err(y, want) < TOL[dtype]


@pytest.mark.parametrize("B,H,N,d,dv,W,dtype,sq,seed", _cases("sliding", 24, 3))
def test_sliding(B, H, N, d, dv, W, dtype, sq, seed):
    K = _kernels()
    q, k, v = rand_qkv(B, H, N, d, dv, seed=seed, dtype=dtype, scale_qk=sq * 2.0)
    y = K.sliding_window_attn(*to_dev(q, k, v), window_size=W, out_dtype=torch.float32)
    want = ref.sliding_dense(q, k, v, window_size=W)
    assert err(y, want) < TOL[dtype]


@pytest.mark.parametrize("B,H,N,d,dv,W,dtype,sq,seed", _cases("identity", 12, 4))
def test_identity(B, H, N, d, dv, W, dtype, sq, seed):
    K = _kernels()
    q, k, v = rand_qkv(B, H, N, d, dv, seed=seed, dtype=dtype, scale_qk=sq)
    y = K.identity_linear_attn(*to_dev(q, k, v), out_dtype=torch.float32)
    want = ref.ref_identity_numerator(q.double(), k.double(), v.double())
    assert err(y, want) < 1e-3


@pytest.mark.parametrize("B,H,N,d,dv,W,dtype,sq,seed", _cases("layer", 10, 5))
def test_layer(B, H, N, d, dv, W, dtype, sq, seed):
    K = _kernels()
    d = min(d, 64)
    q, k, v = rand_qkv(B, H, N, d, dv, seed=seed, dtype=dtype, scale_qk=sq / math.sqrt(math.sqrt(d)))
    q_sw, k_sw, _ = rand_qkv(B, H, N, 32, 1, seed=seed + 7, dtype=dtype, scale_qk=sq)
    dev = to_dev(q, k, v, q_sw, k_sw)
    y = K.based_layer_attn(dev[0], dev[1], dev[2], window_size=W, q_sw=dev[3], k_sw=dev[4])
    want = ref.based_layer_dense(q, k, v, window_size=W, q_sw=q_sw, k_sw=k_sw)
    if dtype == torch.bfloat16:
        from tests.helpers import rounded_err
        assert rounded_err(y, want) < 2e-2
    else:
        assert err(y, want) < 1e-4
