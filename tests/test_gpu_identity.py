"""GPU parity of the identity-map linear attention numerator (la_identity_linear_fwd) against
the oracle's ref_identity_numerator (benchmarks/chunked_attention_benchmark.py:81-93) evaluated
in fp64 on the same bf16 inputs; metric max|y - y_ref| / rms(y_ref)."""

import math

import pytest
import torch

from oracle import reference as ref
from tests.helpers import err, rand_qkv, rounded_err, to_dev

pytestmark = pytest.mark.gpu


def _kernels():
    import kernels
    return kernels


def _want(q, k, v):
    return ref.ref_identity_numerator(q.double(), k.double(), v.double())


@pytest.mark.parametrize("N", [1, 2, 31, 32, 33, 63, 64, 65, 127, 255, 256, 257, 1000])
@pytest.mark.parametrize("d,dv", [(16, 64), (16, 32), (32, 64), (64, 32), (64, 64)])
def test_kernel_shapes(N, d, dv):
    K = _kernels()
    q, k, v = rand_qkv(1, 3, N, d, dv, seed=N * 7 + d + dv, dtype=torch.bfloat16)
    y = K.identity_linear_attn(*to_dev(q, k, v), out_dtype=torch.float32)
    e = err(y, _want(q, k, v))
    assert e < 1e-3, e     # hi + lo bf16 operands: far inside the 2e-2 bar


@pytest.mark.parametrize("d,dv", [(8, 16), (20, 100), (64, 130), (1, 1)])
def test_padded_shapes(d, dv):
    """d and dv outside the kernel's set go through zero-padding and column slices."""
    K = _kernels()
    q, k, v = rand_qkv(2, 2, 150, d, dv, seed=d + dv, dtype=torch.bfloat16)
    y = K.identity_linear_attn(*to_dev(q, k, v), out_dtype=torch.float32)
    assert y.shape == (2, 2, 150, dv)
    assert err(y, _want(q, k, v)) < 1e-3


def test_bf16_output_and_scale():
    K = _kernels()
    q, k, v = rand_qkv(1, 2, 300, 16, 64, seed=4, dtype=torch.bfloat16)
    qd, kd, vd = to_dev(q, k, v)
    y = K.identity_linear_attn(qd, kd, vd)
    assert y.dtype == torch.bfloat16
    assert rounded_err(y, _want(q, k, v)) < 2e-2
    y2 = K.identity_linear_attn(qd, kd, vd, scale=0.5, out_dtype=torch.float32)
    assert err(y2, _want(q, k, v) * (0.5 * math.sqrt(16))) < 1e-3


def test_long_sequence_spot_rows():
    """B2 H16 N8192 d16 dv64: rows spread over the sequence against S_t = sum_{u<=t} k_u v_u^T in
    fp64 (y_t = scale q_t S_t), which checks the block prefixes at full length."""
    K = _kernels()
    B, H, N = 2, 16, 8192
    q, k, v = rand_qkv(B, H, N, 16, 64, seed=99, dtype=torch.bfloat16)
    y = K.identity_linear_attn(*to_dev(q, k, v), out_dtype=torch.float32).cpu()
    for (b, h) in [(0, 0), (1, 15), (0, 7)]:
        kk, vv, qq = k[b, h].double(), v[b, h].double(), q[b, h].double()
        for t in [0, 63, 64, 1000, 4095, 4096, 8191]:
            want = (qq[t] / 4.0) @ (kk[: t + 1].T @ vv[: t + 1])
            got = y[b, h, t].double()
            assert (got - want).abs().max() / want.pow(2).mean().sqrt() < 1e-3, (b, h, t)


def test_errors_raise():
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(1, 1, 8, 16, 16, seed=0, dtype=torch.float32))
    with pytest.raises(RuntimeError):
        K.identity_linear_attn(q, k, v)                                  # fp32
    q2, k2, v2 = to_dev(*rand_qkv(1, 1, 8, 80, 16, seed=0, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError):
        K.identity_linear_attn(q2, k2, v2)                               # d > 64
    e = torch.empty(1, 2, 0, 16, device="cuda", dtype=torch.bfloat16)
    assert K.identity_linear_attn(e, e, e).shape == (1, 2, 0, 16)
