"""GPU parity of the segment-state chunked path (head dims other than 16: d <= 64, dv <= 128,
bf16) against the fp64 oracle.

The path cuts the sequence into 512-token segments: a state kernel writes every segment's
exclusive state prefix in the feature basis (fp16 with per-tile exponents), an output kernel
contracts every query's features with its segment's prefix and adds the quadratic form over
the segment's own keys.  Lengths around the segment and tile boundaries (255/256/257,
511/512/513, 1023/1024/1025) check the hand-over between the two parts.  Bar as for the other
bf16 paths: max|y - y_ref| / rms(y_ref) < 2e-2, fp32 output against fp64 on the same
bf16-rounded inputs.
"""

import pytest
import torch

from oracle import reference as ref
from tests.helpers import err, head_errs, rand_qkv, rounded_err, rows_fp64, to_dev

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _kernels():
    import kernels
    return kernels


@pytest.mark.parametrize("N", [1, 40, 255, 256, 257, 511, 512, 513, 1023, 1024, 1025, 1600, 2500])
@pytest.mark.parametrize("d,dv", [(64, 64), (32, 128), (48, 40), (17, 8), (5, 96)])
def test_general_matches_oracle(N, d, dv):
    K = _kernels()
    q, k, v = rand_qkv(1, 2, N, d, dv, seed=N + 7 * d + dv, dtype=torch.bfloat16, scale_qk=1.0)
    qd, kd, vd = to_dev(q, k, v)
    y = K.based_chunked(qd, kd, vd, out_dtype=torch.float32)
    num = K.based_chunked(qd, kd, vd, normalize=False, out_dtype=torch.float32)
    want, want_num, _ = ref.based_dense(q, k, v)
    e, en = err(y, want), err(num, want_num)
    print(f"N={N} d={d} dv={dv} err={e:.3e} num_err={en:.3e}")
    assert e < TOL and en < TOL


def test_general_wrappers_and_batch():
    """chunked_nki_numerator / chunked_based_attn at d = 64 over six heads: bf16 outputs against
    the oracle (max |y - y_ref| / (|y_ref| + rms), the metric for outputs rounded to bf16), and
    the fp32 numerator against the same call's bf16 output."""
    K = _kernels()
    q, k, v = rand_qkv(2, 3, 1300, 64, 64, seed=11, dtype=torch.bfloat16)
    qd, kd, vd = to_dev(q, k, v)
    want, want_num, _ = ref.based_dense(q, k, v)
    num = K.chunked_nki_numerator(qd, kd, vd, chunk_size=64)
    y = K.chunked_based_attn(qd, kd, vd, chunk_size=64)
    assert num.dtype == torch.bfloat16 and y.dtype == torch.bfloat16
    e_num, e_y = rounded_err(num, want_num), rounded_err(y, want)
    print(f"rounded errs num={e_num:.3e} y={e_y:.3e}")
    assert e_num < TOL and e_y < TOL
    num32 = K.based_chunked(qd, kd, vd, normalize=False, out_dtype=torch.float32)
    assert max(head_errs(num32, want_num)) < TOL
    assert torch.equal(num32.to(torch.bfloat16), num)


@pytest.mark.parametrize("case", ["v_x1e4", "v_x1e-5", "qk_x8", "v_steps"])
def test_general_range(case):
    """Feature, state and value ranges: V scaled by 1e4 and 1e-5, large scores (q, k x 8: |s|
    up to ~150) and V steps of 1e3 between segments (the state prefixes' exponents change)."""
    K = _kernels()
    N, d, dv = 1800, 64, 64
    q, k, v = rand_qkv(1, 2, N, d, dv, seed=5, dtype=torch.float32)
    if case == "v_x1e4":
        v = v * 1e4
    elif case == "v_x1e-5":
        v = v * 1e-5
    elif case == "qk_x8":
        q, k = q * 8, k * 8
    else:
        steps = torch.tensor([1e-2, 10.0, 1e-1, 1e1])
        v = v * steps[(torch.arange(N) // 512).clamp(max=3)].view(1, 1, N, 1)
    q, k, v = (x.to(torch.bfloat16) for x in (q, k, v))
    y = K.based_chunked(*to_dev(q, k, v), out_dtype=torch.float32)
    want, _, _ = ref.based_dense(q, k, v)
    es = head_errs(y, want)
    print(case, [f"{e:.3e}" for e in es])
    assert max(es) < TOL


def test_general_long_d64():
    """B1 H2 N 16384 d64: fp64 rows spread over the sequence (last rows of late segments)."""
    K = _kernels()
    N = 16384
    q, k, v = rand_qkv(1, 2, N, 64, 64, seed=21, dtype=torch.bfloat16)
    y = K.based_chunked(*to_dev(q, k, v), out_dtype=torch.float32).cpu()
    rows = torch.tensor([0, 511, 512, 4000, 8191, 12345, N - 1])
    for h in range(2):
        want = rows_fp64(q, k, v, 0, h, rows)
        e = ref.rel_err(y[0, h, rows], want)
        print(f"head {h} rows err={e:.3e}")
        assert e < TOL


def test_general_d64_many_heads():
    """B2 H16 N4096 d64 dv64 (the reference's chunked head dim over 32 heads): more state
    work-groups than CUs, so two share a CU and the sweep alternates their wave priorities.
    The first 1024 rows of every head against the dense fp64 oracle and rows across the later
    segments of every head against fp64 rows."""
    K = _kernels()
    B, H, N = 2, 16, 4096
    q, k, v = rand_qkv(B, H, N, 64, 64, seed=41, dtype=torch.bfloat16)
    y = K.based_chunked(*to_dev(q, k, v), out_dtype=torch.float32).cpu()
    n = 1024
    want, _, _ = ref.based_dense(q[:, :, :n], k[:, :, :n], v[:, :, :n])
    e0 = max(head_errs(y[:, :, :n], want))
    rows = torch.tensor([1500, 2047, 2048, 3000, 3583, 3584, N - 1])
    e1 = 0.0
    for b in range(B):
        for h in range(H):
            e1 = max(e1, ref.rel_err(y[b, h, rows], rows_fp64(q, k, v, b, h, rows)))
    print(f"general d64 B2 H16 N4096: prefix rows err={e0:.3e}, later rows err={e1:.3e}")
    assert e0 < TOL and e1 < TOL


def test_solution_takes_general_path_for_long_sequences():
    """solution() at d = 32 from GENERAL_CHUNKED_MIN_T tokens runs the segment-state path
    (equal to chunked_based_attn) and matches fp64 rows; below it the fused kernel."""
    K = _kernels()
    from kernels import pytorch_attention
    N = pytorch_attention.GENERAL_CHUNKED_MIN_T
    q, k, v = rand_qkv(1, 1, N, 32, 64, seed=3, dtype=torch.bfloat16)
    qd, kd, vd = to_dev(q, k, v)
    y = K.solution(qd, kd, vd)
    assert torch.equal(y, K.chunked_based_attn(qd, kd, vd))
    y32 = K.based_chunked(qd, kd, vd, out_dtype=torch.float32).cpu()
    rows = torch.tensor([5, 700, N // 2, N - 1])
    assert ref.rel_err(y32[0, 0, rows], rows_fp64(q, k, v, 0, 0, rows)) < TOL
    ys = K.solution(qd[:, :, :300], kd[:, :, :300], vd[:, :, :300])
    assert torch.equal(ys, K.solution_nki(qd[:, :, :300], kd[:, :, :300], vd[:, :, :300]))


TOL_F32 = 1e-4


@pytest.mark.parametrize("N", [1, 100, 511, 512, 513, 1025, 2500])
@pytest.mark.parametrize("d,dv", [(16, 64), (64, 64), (32, 128), (5, 96), (48, 40)])
def test_general_f32_matches_oracle(N, d, dv):
    """fp32 inputs on the segment-state path (fp32 features, states and sums; fp32 MFMAs)
    against the fp64 oracle at the fp32 bar, normalised and numerator."""
    K = _kernels()
    q, k, v = rand_qkv(1, 2, N, d, dv, seed=N + 3 * d + dv, dtype=torch.float32)
    qd, kd, vd = to_dev(q, k, v)
    y = K.based_chunked(qd, kd, vd)
    num = K.based_chunked(qd, kd, vd, normalize=False)
    assert y.dtype == torch.float32
    want, want_num, _ = ref.based_dense(q, k, v)
    e, en = err(y, want), err(num, want_num)
    print(f"fp32 N={N} d={d} dv={dv} err={e:.3e} num_err={en:.3e}")
    assert e < TOL_F32 and en < TOL_F32


def test_general_f32_wrappers():
    """chunked_nki_numerator at fp32 (the reference's chunked kernel takes fp32 inputs,
    kernels/nki_attention_chunked.py:27-33) over six heads, and a bf16 output of fp32 inputs."""
    K = _kernels()
    q, k, v = rand_qkv(2, 3, 1200, 16, 64, seed=4, dtype=torch.float32)
    qd, kd, vd = to_dev(q, k, v)
    want, want_num, _ = ref.based_dense(q, k, v)
    num = K.chunked_nki_numerator(qd, kd, vd, chunk_size=64)
    assert num.dtype == torch.float32 and max(head_errs(num, want_num)) < TOL_F32
    yb = K.based_chunked(qd, kd, vd, out_dtype=torch.bfloat16)
    assert torch.equal(yb, K.based_chunked(qd, kd, vd).to(torch.bfloat16))
