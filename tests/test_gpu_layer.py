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


def _fused(q, k, v, q_sw, k_sw, W, out_dtype):
    """la_based_layer_fwd through the C ABI: the whole layer in one output launch."""
    from kernels import _lib
    L = _lib.lib()
    b, h, t, d = q.shape
    dv, d_sw = v.shape[-1], q_sw.shape[-1]
    out = torch.empty(b, h, t, dv, dtype=out_dtype, device="cuda")
    nb = int(L.la_based_chunked_workspace_bytes_dt(b, h, t, d, dv, 64, 1))
    ws = torch.empty(max(nb, 16), dtype=torch.uint8, device="cuda")
    rc = L.la_based_layer_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), q_sw.data_ptr(), k_sw.data_ptr(),
                              _lib.dtype_code(q.dtype), out.data_ptr(), _lib.dtype_code(out_dtype), b, h, t, d, dv,
                              d_sw, W, 1.0 / math.sqrt(d), 1.0 / math.sqrt(d_sw), 1e-6, ws.data_ptr(), nb,
                              _lib.stream_of(q))
    _lib.check(rc, "la_based_layer_fwd")
    return out


def _layer_inputs(B, H, N, dv, d_sw, seed, vscale=1.0):
    q, k, v = rand_qkv(B, H, N, 16, dv, seed=seed, dtype=torch.float32, scale_qk=0.5)
    q_sw, k_sw, _ = rand_qkv(B, H, N, d_sw, 1, seed=seed + 1, dtype=torch.float32)
    v = v * torch.as_tensor(vscale, dtype=torch.float32)
    return tuple(x.bfloat16() for x in (q, k, v, q_sw, k_sw))


@pytest.mark.parametrize("B,H,N,dv,d_sw,W", [
    (1, 2, 300, 64, 64, 64),     # three one-chunk segments: the 64 keys before each come from the prologue
    (1, 2, 3000, 64, 64, 64),    # 24 segments of one chunk
    (2, 3, 1100, 24, 32, 17),    # dv < 64 (columns past dv), d_sw 32, ragged last chunk
    (1, 1, 700, 8, 16, 1),       # window 1: the diagonal only
    (1, 2, 257, 64, 64, 33),     # window 33: the first key tile is outside every window
    (2, 16, 2048, 64, 64, 64),   # 32 heads, 16 segments each: two per layer work-group
    (2, 16, 1900, 64, 64, 64),   # 15 segments: two per layer work-group, the last one alone
    (1, 1, 9000, 64, 64, 50),    # several chunks per segment
])
def test_fused_layer_matches_oracle(B, H, N, dv, d_sw, W):
    """The one-launch layer against fp64 linear attention + fp64 sliding-window softmax, fp32 and
    bf16 outputs (the bf16 metric relative to |y| + rms)."""
    q, k, v, q_sw, k_sw = _layer_inputs(B, H, N, dv, d_sw, seed=N + dv + W)
    dev = to_dev(q, k, v, q_sw, k_sw)
    want = ref.based_layer_dense(q, k, v, window_size=W, q_sw=q_sw, k_sw=k_sw)
    y32 = _fused(*dev, W, torch.float32)
    yb = _fused(*dev, W, torch.bfloat16)
    e, eb = err(y32, want), rounded_err(yb, want)
    print(f"B{B} H{H} N{N} dv{dv} d_sw{d_sw} W{W}: err={e:.3e} bf16 out={eb:.3e}")
    assert e < 2e-2 and eb < 2e-2


@pytest.mark.parametrize("case", ["v_x1e4", "v_x1e-5", "v_steps"])
def test_fused_layer_v_range(case):
    """V far from N(0, 1): the recurrence's V^T exponent U away from 0 (the softmax branch reads
    that fp16 V^T in the same units), and an exponent that rises inside a segment (the previous
    chunk's V^T then stays in its old units for the window's first keys)."""
    B, H, N, dv, d_sw, W = 1, 1, 9000, 64, 64, 64   # one head: segments of three 128-token chunks
    q, k, v, q_sw, k_sw = _layer_inputs(B, H, N, dv, d_sw, seed=21)
    if case == "v_x1e4":
        v = (v.float() * 1e4).bfloat16()
    elif case == "v_x1e-5":
        v = (v.float() * 1e-5).bfloat16()
    else:
        t = torch.ones(1, 1, N, 1)
        t[:, :, :1000] = 1e-4
        t[:, :, 1450:] = 300.0   # inside a segment's second chunk
        v = (v.float() * t).bfloat16()
    want = ref.based_layer_dense(q, k, v, window_size=W, q_sw=q_sw, k_sw=k_sw)
    y = _fused(*to_dev(q, k, v, q_sw, k_sw), W, torch.float32)
    errs = [ref.rel_err(y[0, hh].cpu(), want[0, hh]) for hh in range(H)]
    print(f"{case}: per-head err " + " ".join(f"{x:.2e}" for x in errs))
    assert max(errs) < 2e-2


def test_fused_layer_v_steps_two_segments_per_work_group():
    """32 heads of 16 one-chunk segments, so that each layer work-group runs two segments from the
    first one's prefix: V 1e-4 for the first 700 tokens and 300 from token 1450 on (inside the
    second segment of a work-group), against the fp64 oracle on four heads."""
    B, H, N, dv, d_sw, W = 2, 16, 2048, 64, 64, 64
    q, k, v, q_sw, k_sw = _layer_inputs(B, H, N, dv, d_sw, seed=23)
    t = torch.ones(1, 1, N, 1)
    t[:, :, :700] = 1e-4
    t[:, :, 1450:] = 300.0
    v = (v.float() * t).bfloat16()
    y = _fused(*to_dev(q, k, v, q_sw, k_sw), W, torch.float32)
    for b, hh in ((0, 0), (0, 7), (1, 8), (1, 15)):
        sl = (slice(b, b + 1), slice(hh, hh + 1))
        want = ref.based_layer_dense(q[sl], k[sl], v[sl], window_size=W, q_sw=q_sw[sl], k_sw=k_sw[sl])
        e = ref.rel_err(y[sl].cpu(), want)
        print(f"v steps, head ({b}, {hh}): err={e:.3e}")
        assert e < 2e-2


def test_fused_layer_b2h16n8192():
    """The benchmark layer (B2 H16 N8192, d 16, d_sw 64, dv 64, window 64) in one output launch:
    two heads against the fp64 oracle over the whole sequence, and the Python entry point
    (based_layer_attn takes the fused kernel for this shape) bit for bit equal to the C-ABI call."""
    K = _kernels()
    B, H, N, dv, d_sw, W = 2, 16, 8192, 64, 64, 64
    q, k, v, q_sw, k_sw = _layer_inputs(B, H, N, dv, d_sw, seed=22)
    dev = to_dev(q, k, v, q_sw, k_sw)
    y = _fused(*dev, W, torch.bfloat16)
    y2 = K.based_layer_attn(dev[0], dev[1], dev[2], window_size=W, q_sw=dev[3], k_sw=dev[4])
    assert torch.equal(y, y2)
    for b, hh in ((0, 0), (1, 15)):
        sl = (slice(b, b + 1), slice(hh, hh + 1))
        want = ref.based_layer_dense(q[sl], k[sl], v[sl], window_size=W, q_sw=q_sw[sl], k_sw=k_sw[sl])
        e = rounded_err(y[sl], want)
        print(f"B2 H16 N8192 head ({b}, {hh}): err={e:.3e}")
        assert e < 2e-2
