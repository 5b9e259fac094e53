"""V with all-zero regions: whole 64-key blocks, 128-token chunks, segments and heads of zeros.

The bf16 kernels store V in fp16 with power-of-two exponents chosen from max |v| of a block,
chunk or head; an all-zero block has no exponent of its own (its max is 0).  These cases hold
every path to finite outputs at its bar against fp64 when parts of V are zero (zero-padded
sequences, masked values), and to exact zeros where all of a head's V is zero.
"""

import pytest
import torch

from oracle import reference as ref
from tests.helpers import head_errs, rand_qkv, rounded_err, to_dev

pytestmark = pytest.mark.gpu

TOL = 2e-2
TOL_F32 = 1e-4


def _kernels():
    import kernels
    return kernels


def _qkv(B, H, N, d, dv, seed, dtype, zero):
    """Inputs with V zero on the token ranges in ``zero`` (all heads), q and k scaled by 1/2."""
    q, k, v = rand_qkv(B, H, N, d, dv, seed=seed, dtype=torch.float32, scale_qk=0.5)
    v = v.clone()
    for a, b in zero:
        v[:, :, a:b] = 0
    return q.to(dtype), k.to(dtype), v.to(dtype)


def _run(path, q, k, v):
    K = _kernels()
    qd, kd, vd = to_dev(q, k, v)
    if path == "parallel":
        return K.based_parallel(qd, kd, vd, out_dtype=torch.float32)
    if path == "chunked":
        return K.based_chunked(qd, kd, vd, out_dtype=torch.float32)
    if path == "sliding":
        return K.sliding_window_attn(qd, kd, vd, window_size=64, out_dtype=torch.float32)
    raise ValueError(path)


# (path, d, dv, dtype, B, H, N): the packed parallel kernel, the register-staged one, the fp32
# three-term kernel, the d = 16 chunk recurrence (one-chunk segments at B1 H2, four-chunk
# segments at B2 H16), the segment-state path (bf16 d64, fp32 d16)
CASES = [
    ("parallel", 16, 64, torch.bfloat16, 1, 2, 1100),
    ("parallel", 32, 64, torch.bfloat16, 1, 2, 1100),
    ("parallel", 16, 64, torch.float32, 1, 3, 777),
    ("chunked", 16, 64, torch.bfloat16, 1, 2, 3000),
    ("chunked", 16, 64, torch.bfloat16, 2, 16, 2600),
    ("chunked", 64, 64, torch.bfloat16, 1, 2, 1500),
    ("chunked", 16, 64, torch.float32, 1, 2, 1500),
]

# zero token ranges: whole 64-key blocks and 128-token chunks inside the sequence; the start of
# the sequence (the first blocks, chunk and segment have no nonzero V before them)
ZEROS = [((64, 320), (1000, 1300)), ((0, 600),)]


@pytest.mark.parametrize("zero", ZEROS, ids=["inner", "leading"])
@pytest.mark.parametrize("path,d,dv,dtype,B,H,N", CASES)
def test_zero_v_regions(path, d, dv, dtype, B, H, N, zero):
    q, k, v = _qkv(B, H, N, d, dv, seed=N + d, dtype=dtype, zero=zero)
    heads = [(0, 0), (B - 1, H - 1)]
    y = _run(path, q, k, v).cpu()
    assert torch.isfinite(y).all(), f"{path} d={d} dv={dv} {dtype}: non-finite outputs"
    tol = TOL_F32 if dtype == torch.float32 else TOL
    for b, h in heads:
        sl = (slice(b, b + 1), slice(h, h + 1))
        want, _, _ = ref.based_dense(q[sl], k[sl], v[sl])
        e = max(head_errs(y[sl], want))
        print(f"{path} d={d} dv={dv} {dtype} B{B} H{H} N{N} zero {zero} head ({b},{h}): err={e:.3e}")
        assert e < tol


def test_zero_v_sliding():
    q, k, v = _qkv(1, 2, 1000, 64, 64, seed=5, dtype=torch.bfloat16, zero=((64, 320),))
    y = _run("sliding", q, k, v).cpu()
    want = ref.sliding_dense(q, k, v, window_size=64)
    e = max(head_errs(y, want))
    print(f"sliding W64 zero V blocks: err={e:.3e}")
    assert torch.isfinite(y).all() and e < TOL


@pytest.mark.parametrize("path,d,dv,dtype,B,H,N", CASES)
def test_zero_v_head(path, d, dv, dtype, B, H, N):
    """Head (0, 0) with V zero everywhere: its outputs are exactly zero; the other heads are
    unaffected."""
    q, k, v = rand_qkv(B, H, N, d, dv, seed=N + 2 * d, dtype=torch.float32, scale_qk=0.5)
    v = v.clone()
    v[0, 0] = 0
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    y = _run(path, q, k, v).cpu()
    assert torch.isfinite(y).all(), f"{path} d={d} dv={dv} {dtype}: non-finite outputs"
    assert y[0, 0].abs().max().item() == 0.0
    b, h = B - 1, H - 1
    if (b, h) != (0, 0):
        sl = (slice(b, b + 1), slice(h, h + 1))
        want, _, _ = ref.based_dense(q[sl], k[sl], v[sl])
        e = max(head_errs(y[sl], want))
        tol = TOL_F32 if dtype == torch.float32 else TOL
        print(f"{path} d={d} dv={dv} {dtype} zero head (0,0); head ({b},{h}) err={e:.3e}")
        assert e < tol


def test_zero_v_layer():
    """The one-launch layer (chunk recurrence + sliding window) with zero V blocks and a zero
    leading segment."""
    K = _kernels()
    q, k, v = _qkv(2, 4, 2600, 16, 64, seed=21, dtype=torch.bfloat16, zero=((0, 600), (1000, 1300)))
    g = torch.Generator().manual_seed(22)
    qs = (torch.randn(2, 4, 2600, 16, generator=g) * 0.5).bfloat16()
    ks = (torch.randn(2, 4, 2600, 16, generator=g) * 0.5).bfloat16()
    qd, kd, vd, qsd, ksd = to_dev(q, k, v, qs, ks)
    y = K.based_layer_attn(qd, kd, vd, window_size=64, q_sw=qsd, k_sw=ksd).float().cpu()
    assert torch.isfinite(y).all()
    want = ref.based_layer_dense(q[:, :1], k[:, :1], v[:, :1], window_size=64, q_sw=qs[:, :1], k_sw=ks[:, :1])
    # bf16 output: the rounding alone is 1.7e-2 of the rms here (rows after the zero prefix
    # reach five times the rms), so the bar is taken relative to |y_ref| + rms
    e = rounded_err(y[:, :1], want)
    print(f"layer with zero V regions: err={e:.3e}")
    assert e < TOL


def test_zero_v_identity():
    """Identity-map numerator (bf16 hi + lo operands, no V exponent) with zero V regions."""
    q, k, v = _qkv(1, 2, 1000, 16, 64, seed=9, dtype=torch.bfloat16, zero=((0, 300), (500, 700)))
    y = _kernels().identity_linear_attn(*to_dev(q, k, v), out_dtype=torch.float32).cpu()
    want = ref.ref_identity_numerator(q.double(), k.double(), v.double())
    e = max(head_errs(y, want))
    print(f"identity with zero V regions: err={e:.3e}")
    assert torch.isfinite(y).all() and e < 1e-3


@pytest.mark.parametrize("which", ["q", "k"])
@pytest.mark.parametrize("path,d,dv,dtype,B,H,N", CASES)
def test_zero_q_or_k(path, d, dv, dtype, B, H, N, which):
    """q or k zero everywhere (every score 0, p = 1: each output row is the running mean of v)."""
    q, k, v = rand_qkv(B, H, N, d, dv, seed=N + 3 * d, dtype=torch.float32, scale_qk=0.5)
    if which == "q":
        q = torch.zeros_like(q)
    else:
        k = torch.zeros_like(k)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    y = _run(path, q, k, v).cpu()
    assert torch.isfinite(y).all(), f"{path} d={d} dv={dv} {dtype} zero {which}: non-finite outputs"
    b, h = B - 1, H - 1
    sl = (slice(b, b + 1), slice(h, h + 1))
    want, _, _ = ref.based_dense(q[sl], k[sl], v[sl])
    e = max(head_errs(y[sl], want))
    tol = TOL_F32 if dtype == torch.float32 else TOL
    print(f"{path} d={d} dv={dv} {dtype} zero {which}: err={e:.3e}")
    assert e < tol
