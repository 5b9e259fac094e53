"""GPU parity of the full BASED layer (linear attention + sliding-window softmax,
kernels/nki_attention_sliding.py:4-5) and of the sliding kernel's fused addend
(la_sliding_window_fwd_add) that sums the two branches."""

import math

import pytest
import torch

from oracle import reference as ref
from tests.helpers import err, rand_qkv, rounded_err, to_dev

pytestmark = pytest.mark.gpu


def _kernels():
    import kernels
    return kernels


@pytest.mark.parametrize("t,d,d_sw,dv,W,dtype", [
    (300, 16, 64, 64, 64, torch.bfloat16),    # chunked linear branch, resident sliding kernel
    (100, 16, None, 64, 37, torch.bfloat16),  # fused linear branch, shared projections
    (257, 16, 16, 17, 5, torch.bfloat16),     # dv not a multiple of 4: scalar stores
    (300, 32, 32, 48, 200, torch.bfloat16),   # d = 32: fused linear branch; streaming sliding kernel
    (129, 16, 32, 32, 65, torch.float32),     # fp32 kernels
])
def test_layer_matches_oracle(t, d, d_sw, dv, W, dtype):
    K = _kernels()
    q, k, v = rand_qkv(1, 2, t, d, dv, seed=t + d, dtype=dtype, scale_qk=0.5)
    if d_sw is None:
        q_sw = k_sw = None
    else:
        q_sw, k_sw, _ = rand_qkv(1, 2, t, d_sw, 1, seed=t + d_sw + 1, dtype=dtype)
    dev = to_dev(q, k, v) + ((None, None) if d_sw is None else to_dev(q_sw, k_sw))
    y = K.based_layer_attn(*dev[:3], window_size=W, q_sw=dev[3], k_sw=dev[4])
    assert y.dtype == dtype and y.shape == (1, 2, t, dv)
    want = ref.based_layer_dense(q, k, v, window_size=W, q_sw=q_sw, k_sw=k_sw)
    if dtype == torch.bfloat16:
        assert rounded_err(y, want) < 2e-2
    else:
        assert err(y, want) < 1e-4


@pytest.mark.parametrize("N,d,dv,W,dtype", [
    (300, 64, 64, 64, torch.bfloat16),   # resident kernel
    (300, 16, 48, 100, torch.bfloat16),  # streaming kernel, vector stores
    (130, 16, 17, 9, torch.bfloat16),    # streaming kernel, scalar stores
    (130, 16, 32, 64, torch.float32),    # fp32 kernel
])
def test_fused_addend_is_exact(N, d, dv, W, dtype):
    """sliding + addend in the kernel's store equals the fp32 sliding output plus the addend
    computed apart, bit for bit (one fp32 add, then one rounding); the addend is not modified."""
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(2, 2, N, d, dv, seed=N + dv, dtype=dtype, scale_qk=0.7))
    g = torch.Generator(device="cuda").manual_seed(5)
    add = torch.randn(2, 2, N, dv, device="cuda", generator=g)
    add_copy = add.clone()
    base = K.sliding_window_attn(q, k, v, window_size=W, out_dtype=torch.float32)
    y32 = K.sliding_window_attn(q, k, v, window_size=W, out_dtype=torch.float32, addend=add)
    assert torch.equal(y32, base + add)
    y = K.sliding_window_attn(q, k, v, window_size=W, addend=add)
    assert y.dtype == dtype and torch.equal(y, (base + add).to(dtype))
    assert torch.equal(add, add_copy)


def test_layer_in_place_fp32_sum_and_empty():
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(1, 1, 70, 16, 32, seed=3, dtype=torch.float32))
    lin = K.based_parallel(q, k, v, out_dtype=torch.float32)
    sw = K.sliding_window_attn(q, k, v, window_size=64, out_dtype=torch.float32)
    assert torch.equal(K.based_layer_attn(q, k, v, window_size=64), lin + sw)
    e = torch.empty(1, 2, 0, 16, device="cuda", dtype=torch.bfloat16)
    assert K.based_layer_attn(e, e, e).shape == (1, 2, 0, 16)


def test_layer_argument_errors():
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(1, 1, 8, 16, 16, seed=0, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError):
        K.based_layer_attn(q, k, v, window_size=0)
    with pytest.raises(RuntimeError):
        K.based_layer_attn(q, k, v, q_sw=q[:, :, :4], k_sw=k[:, :, :4])   # t differs from v's
    with pytest.raises(RuntimeError):
        K.based_layer_attn(q, k, v, q_sw=q.float(), k_sw=k.float())       # dtype differs
    with pytest.raises(RuntimeError):
        K.sliding_window_attn(q, k, v, addend=torch.zeros(1, 1, 8, 8, device="cuda"))   # shape
