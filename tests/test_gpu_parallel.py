"""GPU parity of the fused parallel BASED kernel (la_based_parallel_fwd) against the oracle.

The kernel's fp32 output is compared with the oracle evaluated in fp64 on the same
dtype-rounded inputs; metric max|y - y_ref| / rms(y_ref); bars 2e-2 (bf16 inputs) and 1e-4
(fp32 inputs).
"""

import math

import pytest
import torch

from oracle import reference as ref
from tests.helpers import err, head_errs, load_golden, rand_qkv, rounded_err, to_dev

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
TOL_F32 = 1e-4


def _kernels():
    import kernels
    return kernels


@pytest.mark.parametrize("name", ["based_b1h2n67d16dv64", "based_b1h1n130d16dv16", "based_b1h2n129d4dv8",
                                  "based_b1h2n67d16dv64_unscaled"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_golden(name, dtype):
    K = _kernels()
    g = load_golden(name)
    q, k, v = (torch.from_numpy(g[x]) for x in "qkv")
    qd, kd, vd = to_dev(q, k, v, dtype=dtype)
    y, den = K.based_parallel(qd, kd, vd, out_dtype=torch.float32, return_den=True)
    torch.cuda.synchronize()
    tol = TOL_BF16 if dtype == torch.bfloat16 else TOL_F32
    e = err(y, torch.from_numpy(g["y"]))
    print(f"{name} {dtype} err={e:.3e}")
    assert e < tol
    assert err(den, torch.from_numpy(g["den"])) < (TOL_BF16 if dtype == torch.bfloat16 else 1e-5)


@pytest.mark.parametrize("N", [1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 511, 700])
def test_ragged_lengths_bf16(N):
    K = _kernels()
    q, k, v = rand_qkv(1, 3, N, 16, 64, seed=N, dtype=torch.bfloat16, scale_qk=0.5)
    y = K.based_parallel(*to_dev(q, k, v), out_dtype=torch.float32)
    want, _, _ = ref.based_dense(q, k, v)
    assert err(y, want) < TOL_BF16


@pytest.mark.parametrize("d,dv", [(1, 1), (4, 8), (8, 16), (16, 17), (16, 32), (24, 40), (32, 64), (64, 64),
                                  (64, 96), (128, 128), (16, 128), (100, 3)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_head_dims(d, dv, dtype):
    K = _kernels()
    N = 200
    q, k, v = rand_qkv(2, 2, N, d, dv, seed=d * 1000 + dv, dtype=dtype, scale_qk=1.0 / math.sqrt(math.sqrt(d)))
    y = K.based_parallel(*to_dev(q, k, v), out_dtype=torch.float32)
    want, _, _ = ref.based_dense(q, k, v)
    e = err(y, want)
    print(f"d={d} dv={dv} {dtype} err={e:.3e}")
    assert e < (TOL_BF16 if dtype == torch.bfloat16 else TOL_F32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_numerator_and_den(dtype):
    K = _kernels()
    q, k, v = rand_qkv(1, 2, 300, 16, 64, seed=7, dtype=dtype, scale_qk=0.5)
    num, den = K.based_parallel(*to_dev(q, k, v), normalize=False, out_dtype=torch.float32, return_den=True)
    _, want_num, want_den = ref.based_dense(q, k, v)
    assert err(num, want_num) < (TOL_BF16 if dtype == torch.bfloat16 else TOL_F32)
    assert err(den, want_den) < 1e-3


def test_bf16_output_is_rounded_fp32_output():
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(2, 2, 333, 16, 64, seed=3, dtype=torch.bfloat16))
    y32 = K.based_parallel(q, k, v, out_dtype=torch.float32)
    y16 = K.solution_nki(q, k, v)
    assert y16.dtype == torch.bfloat16
    assert torch.equal(y16, y32.to(torch.bfloat16))


def test_parallel_fp32_b1h4n1024():
    K = _kernels()
    cfg = ref.CONFIGS["parallel_fp32_b1h4n1024"]
    q, k, v = ref.config_inputs(cfg)
    y = K.solution_nki(*to_dev(q, k, v))
    assert y.dtype == torch.float32
    want, _, _ = ref.based_dense(q, k, v)
    e = err(y, want)
    print(f"parallel fp32 B1 H4 N1024 err={e:.3e}")
    assert e < TOL_F32


@pytest.mark.parametrize("prescale", [True, False])
def test_parallel_bf16_b2h16n2048(prescale):
    K = _kernels()
    cfg = ref.CONFIGS["parallel_bf16_b2h16n2048"]
    q, k, v = ref.config_inputs(cfg, prescale=prescale)
    y = K.based_parallel(*to_dev(q, k, v), out_dtype=torch.float32)
    want, _, _ = ref.based_dense(q, k, v)
    e = err(y, want)
    print(f"parallel bf16 B2 H16 N2048 prescale={prescale} err={e:.3e}")
    assert e < TOL_BF16


def test_b2_h16_n8192_prefix_and_spot_rows():
    """B2 H16 N8192 d16 dv64 bf16 (the headline workload): every row of every head against the
    oracle's fp64 chunk recurrence (pinned against the dense form for any chunk size), plus the
    first 2048 rows against the dense oracle (causal prefix invariance makes the prefix
    self-contained) and the last rows of two heads by a direct fp64 evaluation."""
    K = _kernels()
    q, k, v = ref.make_inputs(2, 16, 8192, 16, 64, torch.bfloat16, seed=2)
    y = K.based_parallel(*to_dev(q, k, v), out_dtype=torch.float32).cpu()
    want_all = ref.based_chunked(q, k, v, chunk=512, dtype=torch.float64)
    e_all = max(head_errs(y, want_all))
    print(f"parallel B2 H16 N8192 all rows: worst head err={e_all:.3e}")
    assert e_all < TOL_BF16
    n = 2048
    want, _, _ = ref.based_dense(q[:, :, :n], k[:, :, :n], v[:, :, :n])
    assert err(y[:, :, :n], want) < TOL_BF16
    for (b, h) in [(0, 0), (1, 15)]:
        qq, kk, vv = q[b, h].double(), k[b, h].double(), v[b, h].double()
        rows = torch.arange(8192 - 64, 8192)
        s = (qq[rows] / 4.0) @ kk.T
        p = (1 + s + 0.5 * s * s) * (torch.arange(8192).unsqueeze(0) <= rows.unsqueeze(1))
        want_rows = (p @ vv) / (p.sum(-1, keepdim=True) + 1e-6)
        e = ref.rel_err(y[b, h, rows], want_rows)
        assert e < TOL_BF16, e


@pytest.mark.parametrize("B,H,N", [(2, 16, 4096), (1, 8, 16384)])
def test_parallel_256_query_orders_all_rows(B, H, N):
    """The 256-query kernel's work-group orders: B2 H16 N4096 holds exactly one first round of
    two work-groups per CU (its second half taken in reverse), B1 H8 N16384 more blocks per XCD
    than that.  Every row of every head against the oracle's fp64 chunk recurrence."""
    K = _kernels()
    q, k, v = ref.make_inputs(B, H, N, 16, 64, torch.bfloat16, seed=N + H)
    y = K.based_parallel(*to_dev(q, k, v), out_dtype=torch.float32).cpu()
    want = ref.based_chunked(q, k, v, chunk=512, dtype=torch.float64)
    e = max(head_errs(y, want))
    print(f"parallel B{B} H{H} N{N} all rows: worst head err={e:.3e}")
    assert e < TOL_BF16


def test_fp32_tiled_kernel_b2_h16_n8192_all_rows():
    """fp32 B2 H16 N8192 d16 dv64 (the tiled three-term kernel, two work-groups per CU in the
    paired first-round order): every row of every head against the oracle's fp64 chunk
    recurrence at the fp32 bar."""
    K = _kernels()
    q, k, v = ref.make_inputs(2, 16, 8192, 16, 64, torch.float32, seed=8)
    y = K.based_parallel(*to_dev(q, k, v), out_dtype=torch.float32).cpu()
    want = ref.based_chunked(q, k, v, chunk=512, dtype=torch.float64)
    e = max(head_errs(y, want))
    print(f"fp32 tiled B2 H16 N8192 all rows: worst head err={e:.3e}")
    assert e < TOL_F32


def test_dtype_and_layout_handling():
    K = _kernels()
    q, k, v = rand_qkv(1, 2, 100, 16, 32, seed=9, dtype=torch.float16)
    qd, kd, vd = to_dev(q, k, v)
    y = K.solution(qd, kd, vd)
    assert y.dtype == torch.float16 and y.shape == (1, 2, 100, 32)
    want, _, _ = ref.based_dense(q, k, v)
    assert err(y.float(), want) < 1e-2   # output rounded to fp16
    # non-contiguous views are accepted
    qt = qd.transpose(1, 2).contiguous().transpose(1, 2)
    y2 = K.solution(qt, kd, vd)
    assert torch.equal(y, y2)


def test_errors_raise():
    K = _kernels()
    q, k, v = rand_qkv(1, 1, 8, 16, 16, seed=0, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        K.solution_nki(q, k, v)   # CPU tensors: no host path
    qd, kd, vd = to_dev(q, k, v)
    with pytest.raises(RuntimeError):
        K.solution_nki(qd, kd[:, :, :4], vd)
    with pytest.raises(RuntimeError):
        K.based_parallel(qd, kd, vd, scale=-1.0)
    qd2 = torch.randn(1, 1, 8, 130, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        K.solution_nki(qd2, qd2, vd)   # d > 128 unsupported


def test_empty_sequence():
    K = _kernels()
    q = torch.empty(1, 2, 0, 16, device="cuda", dtype=torch.bfloat16)
    v = torch.empty(1, 2, 0, 64, device="cuda", dtype=torch.bfloat16)
    y = K.solution_nki(q, q, v)
    assert y.shape == (1, 2, 0, 64)


def test_single_hip_runtime_and_native_library():
    from kernels import _lib
    _lib.lib()
    rts = _lib.hip_runtimes_loaded()
    print("HIP runtimes mapped:", rts)
    assert len(rts) == 1


@pytest.mark.parametrize("B,H,N,dv", [(1, 2, 777, 64), (2, 8, 1024, 32)])
def test_pack_then_packed_kernel_equals_fused_call(B, H, N, dv):
    """la_based_parallel_pack + la_based_parallel_fwd_packed is la_based_parallel_fwd, bit for
    bit, including a second k and v packed into the same workspace."""
    from kernels import _lib
    L = _lib.lib()
    d = 16
    ws_bytes = int(L.la_based_parallel_workspace_bytes(B, H, N, d, dv, 1))
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    for seed in (11, 12):
        q, k, v = to_dev(*rand_qkv(B, H, N, d, dv, seed=seed, dtype=torch.bfloat16, scale_qk=0.5))
        outs = []
        for mode in ("fused", "split"):
            out = torch.empty(B, H, N, dv, dtype=torch.float32, device="cuda")
            den = torch.empty(B, H, N, dtype=torch.float32, device="cuda")
            args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), 1, out.data_ptr(), 0, den.data_ptr(), B, H, N, d, dv,
                    0.25, 1e-6, 1, ws.data_ptr(), ws_bytes, st)
            if mode == "fused":
                assert L.la_based_parallel_fwd(*args) == 0
            else:
                assert L.la_based_parallel_pack(k.data_ptr(), v.data_ptr(), 1, B, H, N, d, dv, ws.data_ptr(),
                                                ws_bytes, st) == 0
                assert L.la_based_parallel_fwd_packed(*args) == 0
            outs.append((out, den))
        torch.cuda.synchronize()
        assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
        want, _, want_den = ref.based_dense(q.cpu(), k.cpu(), v.cpu())
        assert err(outs[1][0], want) < TOL_BF16
        assert err(outs[1][1], want_den) < TOL_BF16


@pytest.mark.parametrize("N,d,dv,dtype", [(255, 16, 64, torch.bfloat16), (256, 16, 64, torch.bfloat16),
                                          (1000, 16, 32, torch.bfloat16), (300, 32, 64, torch.bfloat16),
                                          (300, 16, 64, torch.float32)])
def test_solution_dispatch_by_length(N, d, dv, dtype):
    """solution() runs the chunked kernel from CHUNKED_MIN_T on (bf16, d = 16, dv <= 64) and the
    fused kernel otherwise; either way it matches the oracle."""
    K = _kernels()
    from kernels import chunked_attention, pytorch_attention
    q, k, v = rand_qkv(1, 2, N, d, dv, seed=N + d, dtype=dtype, scale_qk=0.5)
    qd, kd, vd = to_dev(q, k, v)
    y = K.solution(qd, kd, vd)
    chunked = N >= pytorch_attention.CHUNKED_MIN_T and chunked_attention.chunked_supported(d, dv, qd.dtype)
    same = chunked_attention.chunked_based_attn(qd, kd, vd) if chunked else K.solution_nki(qd, kd, vd)
    assert torch.equal(y, same)
    want, _, _ = ref.based_dense(q, k, v)
    if dtype == torch.bfloat16:
        assert rounded_err(y, want) < TOL_BF16     # bf16 output
    else:
        assert err(y, want) < TOL_F32


@pytest.mark.parametrize("B,H,N,dv", [(8, 32, 300, 64), (8, 32, 600, 32), (8, 32, 257, 32), (1, 2, 777, 64),
                                      (1, 3, 129, 32)])
def test_packed_work_group_sizes(B, H, N, dv):
    """The packed kernel runs 256-query work-groups when they fill every CU's slots (two per CU
    at dv = 64, three at dv = 32: the first two shapes at 256 CUs) and 128-query ones below that;
    ragged N in both."""
    K = _kernels()
    q, k, v = rand_qkv(B, H, N, 16, dv, seed=N + dv + H, dtype=torch.bfloat16, scale_qk=0.5)
    y, den = K.based_parallel(*to_dev(q, k, v), out_dtype=torch.float32, return_den=True)
    want, _, want_den = ref.based_dense(q, k, v)
    assert err(y, want) < TOL_BF16
    assert err(den, want_den) < TOL_BF16


@pytest.mark.parametrize("B,H,N,d,dv", [(1, 4, 1024, 16, 64), (1, 1, 300, 16, 100), (1, 2, 1000, 32, 128),
                                        (2, 3, 257, 8, 24), (1, 1, 129, 4, 1)])
def test_fp32_key_split(B, H, N, d, dv):
    """fp32 inputs on small grids: shapes outside the three-term kernel (dv 100, 128, d 32, dv 1)
    run every (query block, 64-key block) as its own work-group and add the partial numerators and
    row sums in a second kernel; d <= 16, dv <= 64 with 16-byte rows (the first and fourth shapes)
    run the three-term kernel.  Output, numerator and den against fp64 (dv 100 and 128 the widest
    partials, dv 24 and 1 columns past dv in them; 300 and 257 tokens a ragged last query block,
    whose last key block may lie past N)."""
    K = _kernels()
    L = _lib_mod().lib()
    need = L.la_based_parallel_workspace_bytes(B, H, N, d, dv, 0)
    nqb = (N + 127) // 128
    cols = 32 if dv <= 32 else (64 if dv <= 64 else 128)
    assert need == B * H * nqb * (nqb + 1) * 128 * (cols + 1) * 4   # the split is in use
    q, k, v = rand_qkv(B, H, N, d, dv, seed=N + dv, dtype=torch.float32, scale_qk=1.0 / math.sqrt(math.sqrt(d)))
    want, want_num, want_den = ref.based_dense(q, k, v)
    y, den = K.based_parallel(*to_dev(q, k, v), out_dtype=torch.float32, return_den=True)
    num = K.based_parallel(*to_dev(q, k, v), normalize=False, out_dtype=torch.float32)
    yb = K.based_parallel(*to_dev(q, k, v), out_dtype=torch.bfloat16)
    e, en, ed = err(y, want), err(num, want_num), err(den, want_den)
    print(f"B{B} H{H} N{N} d{d} dv{dv}: err={e:.2e} num={en:.2e} den={ed:.2e}")
    assert e < TOL_F32 and en < TOL_F32 and ed < 1e-5
    assert rounded_err(yb.float(), want) < 1e-2


def _lib_mod():
    from kernels import _lib
    return _lib


@pytest.mark.parametrize("N,d,dv", [(129, 16, 64), (200, 4, 8), (777, 12, 36), (1024, 8, 64), (1000, 16, 32),
                                    (300, 16, 4), (2047, 16, 64)])
def test_fp32_small_grid_three_term_kernel(N, d, dv):
    """fp32 on small grids (d <= 16, dv <= 64, aligned rows): three-term bf16 products.  Normalised
    output, numerator and row sums against fp64 at the fp32 bar; a bf16 output equal to the
    rounded fp32 one; and a misaligned output (the key-split kernel with its combine) equal to the
    fp32 bar too."""
    K = _kernels()
    q, k, v = rand_qkv(1, 3, N, d, dv, seed=N + d + dv, dtype=torch.float32, scale_qk=1.0)
    qd, kd, vd = to_dev(q, k, v)
    want, want_num, want_den = ref.based_dense(q, k, v)
    y, den = K.based_parallel(qd, kd, vd, out_dtype=torch.float32, return_den=True)
    num = K.based_parallel(qd, kd, vd, normalize=False, out_dtype=torch.float32)
    e, en, ed = err(y, want), err(num, want_num), err(den, want_den)
    print(f"fp32 small grid N={N} d={d} dv={dv} err={e:.3e} num={en:.3e} den={ed:.3e}")
    assert e < TOL_F32 and en < TOL_F32 and ed < TOL_F32
    yb = K.based_parallel(qd, kd, vd, out_dtype=torch.bfloat16)
    assert torch.equal(yb, y.to(torch.bfloat16))
    # an output 4 bytes off 16-byte alignment takes the key-split kernel
    buf = torch.empty(y.numel() + 1, dtype=torch.float32, device="cuda")
    y2 = buf[1:].view_as(y)
    from kernels import _lib
    L = _lib.lib()
    B, H = 1, 3
    ws_bytes = int(L.la_based_parallel_workspace_bytes(B, H, N, d, dv, 0))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    rc = L.la_based_parallel_fwd(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), 0, y2.data_ptr(), 0, 0, B, H, N, d, dv,
                                 1.0 / math.sqrt(d), 1e-6, 1, ws.data_ptr(), ws_bytes,
                                 torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert err(y2, want) < TOL_F32


@pytest.mark.parametrize("B,H,N,dv", [(2, 64, 1024, 64), (1, 128, 1100, 32)])
def test_fp32_large_grid_tiled_kernel(B, H, N, dv):
    """fp32 grids whose 256-query blocks fill every CU twice run the tiled three-term kernel (key
    tiles shared by 8 waves through LDS, work-groups in the paired first-round order at dv = 64):
    output and den of every head against fp64, ragged N."""
    K = _kernels()
    d = 16
    q, k, v = rand_qkv(B, H, N, d, dv, seed=N + H, dtype=torch.float32, scale_qk=1.0)
    y, den = K.based_parallel(*to_dev(q, k, v), out_dtype=torch.float32, return_den=True)
    y, den = y.cpu(), den.cpu()
    want, _, want_den = ref.based_dense(q, k, v)
    worst = (0.0, 0.0, None)
    for bb in range(B):
        for hh in range(H):
            sl = (slice(bb, bb + 1), slice(hh, hh + 1))
            e, ed = err(y[sl], want[sl]), err(den[sl], want_den[sl])
            if max(e, ed) > max(worst[0], worst[1]):
                worst = (e, ed, (bb, hh))
    print(f"tiled fp32 B{B} H{H} N{N} dv{dv}: worst head {worst[2]} err={worst[0]:.3e} den={worst[1]:.3e}")
    assert worst[0] < TOL_F32 and worst[1] < TOL_F32
