"""GPU parity of the chunked recurrent BASED kernel (la_based_chunked_fwd) against the oracle.

Bars as for the parallel kernel: max|y - y_ref| / rms(y_ref) below 2e-2 for bf16 inputs,
computed on the fp32 output against the fp64 oracle on the same bf16-rounded inputs.  At full
size (N = 8192, 65536) every row of every head is compared with the oracle's fp64 chunk
recurrence (itself pinned against the dense form), and the checks also use causal prefix
invariance (the first rows against the dense oracle on the prefix), direct fp64 evaluation of
the last rows of some heads, and the exported final state against its closed form
sum_u phi(k_u) [v_u | 1].
"""

import math

import pytest
import torch

from oracle import reference as ref
from tests.helpers import err, head_errs, load_golden, rand_qkv, to_dev

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _kernels():
    import kernels
    return kernels


def _rows_fp64(q, k, v, b, h, rows, eps=1e-6, normalize=True):
    qq, kk, vv = q[b, h].double(), k[b, h].double(), v[b, h].double()
    d = qq.shape[-1]
    s = (qq[rows] / math.sqrt(d)) @ kk.T
    mask = torch.arange(qq.shape[0]).unsqueeze(0) <= rows.unsqueeze(1)
    p = (1 + s + 0.5 * s * s) * mask
    num = p @ vv
    return num / (p.sum(-1, keepdim=True) + eps) if normalize else num


@pytest.mark.parametrize("name", ["based_b1h2n67d16dv64", "based_b1h1n130d16dv16",
                                  "based_b1h2n67d16dv64_unscaled"])
def test_golden(name):
    K = _kernels()
    g = load_golden(name)
    q, k, v = (torch.from_numpy(g[x]) for x in "qkv")
    qd, kd, vd = to_dev(q, k, v, dtype=torch.bfloat16)
    y = K.based_chunked(qd, kd, vd, out_dtype=torch.float32)
    e = err(y, torch.from_numpy(g["y"]))
    num = K.based_chunked(qd, kd, vd, normalize=False, out_dtype=torch.float32)
    en = err(num, torch.from_numpy(g["num"]))
    print(f"{name} err={e:.3e} num_err={en:.3e}")
    assert e < TOL and en < TOL


@pytest.mark.parametrize("N", [1, 2, 63, 64, 65, 127, 128, 129, 200, 511, 1000, 3000])
@pytest.mark.parametrize("dv", [64, 16, 40])
def test_ragged(N, dv):
    K = _kernels()
    q, k, v = rand_qkv(1, 2, N, 16, dv, seed=N + dv, dtype=torch.bfloat16, scale_qk=0.5)
    y = K.based_chunked(*to_dev(q, k, v), out_dtype=torch.float32)
    want, want_num, _ = ref.based_dense(q, k, v)
    e = err(y, want)
    num = K.based_chunked(*to_dev(q, k, v), normalize=False, out_dtype=torch.float32)
    en = err(num, want_num)
    print(f"N={N} dv={dv} err={e:.3e} num_err={en:.3e}")
    assert e < TOL and en < TOL


@pytest.mark.parametrize("B,H", [(1, 1), (2, 3), (1, 8), (2, 16)])
def test_heads_and_segments(B, H):
    """Different B*H change the segment split; the result must not."""
    K = _kernels()
    q, k, v = rand_qkv(B, H, 1500, 16, 64, seed=B * 100 + H, dtype=torch.bfloat16, scale_qk=0.5)
    y = K.based_chunked(*to_dev(q, k, v), out_dtype=torch.float32)
    want, _, _ = ref.based_dense(q, k, v)
    e = err(y, want)
    print(f"B={B} H={H} err={e:.3e}")
    assert e < TOL


def test_matches_parallel_kernel():
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(2, 4, 2500, 16, 64, seed=77, dtype=torch.bfloat16))
    yc = K.based_chunked(q, k, v, out_dtype=torch.float32)
    yp = K.based_parallel(q, k, v, out_dtype=torch.float32)
    e = ref.rel_err(yc.cpu(), yp.cpu())
    print(f"chunked vs parallel err={e:.3e}")
    assert e < 1e-2


def test_reference_wrapper_signatures():
    K = _kernels()
    q, k, v = rand_qkv(1, 2, 300, 16, 16, seed=5, dtype=torch.bfloat16, scale_qk=0.5)
    qd, kd, vd = to_dev(q, k, v)
    num = K.chunked_nki_numerator(qd, kd, vd, chunk_size=64)
    assert num.dtype == torch.bfloat16 and num.shape == (1, 2, 300, 16)
    _, want_num, _ = ref.based_dense(q, k, v)
    assert err(num.float(), want_num) < 2e-2
    y = K.chunked_based_attn(qd, kd, vd, chunk_size=128)
    want, _, _ = ref.based_dense(q, k, v)
    assert err(y.float(), want) < 3e-2


def test_final_state_closed_form():
    K = _kernels()
    q, k, v = rand_qkv(1, 2, 777, 16, 24, seed=9, dtype=torch.bfloat16, scale_qk=0.7)
    _, st = K.based_chunked(*to_dev(q, k, v), out_dtype=torch.float32, return_state=True)
    phik = ref.taylor_feature_map(k.double())
    want = torch.cat([phik.transpose(-2, -1) @ v.double(), phik.sum(-2).unsqueeze(-1)], dim=-1)
    e = ref.rel_err(st.cpu(), want)
    print(f"state err={e:.3e}")
    assert e < 1e-2


@pytest.mark.parametrize("prescale", [True, False])
def test_chunked_b2h16n8192(prescale):
    """Every row of every head against the oracle's fp64 chunk recurrence (pinned against the
    dense form for any chunk size), the first rows against the dense oracle and the last rows
    of three heads by a direct fp64 evaluation."""
    K = _kernels()
    cfg = ref.CONFIGS["chunked_bf16_b2h16n8192"]
    q, k, v = ref.config_inputs(cfg, prescale=prescale)
    y = K.based_chunked(*to_dev(q, k, v), chunk_size=cfg.chunk, out_dtype=torch.float32).cpu()
    want_all = ref.based_chunked(q, k, v, chunk=512, dtype=torch.float64)
    e0 = max(head_errs(y, want_all))
    n = 1024
    want, _, _ = ref.based_dense(q[:, :, :n], k[:, :, :n], v[:, :, :n])
    e1 = err(y[:, :, :n], want)
    rows = torch.arange(cfg.N - 64, cfg.N)
    e2 = max(ref.rel_err(y[b, h, rows], _rows_fp64(q, k, v, b, h, rows)) for b, h in [(0, 0), (0, 7), (1, 15)])
    print(f"chunked B2 H16 N8192 prescale={prescale} all rows worst head err={e0:.3e} prefix err={e1:.3e} "
          f"tail err={e2:.3e}")
    assert e0 < TOL and e1 < TOL and e2 < TOL


def test_chunked_bf16_b1h16n65536():
    """Every row of all 16 heads against the oracle's fp64 chunk recurrence, the first rows
    against the dense oracle, spot rows by a direct fp64 evaluation and the exported state
    against its closed form."""
    K = _kernels()
    cfg = ref.CONFIGS["chunked_bf16_b1h16n65536"]
    q, k, v = ref.config_inputs(cfg)
    y, st = K.based_chunked(*to_dev(q, k, v), chunk_size=cfg.chunk, out_dtype=torch.float32, return_state=True)
    y = y.cpu()
    e0 = 0.0
    for h0 in range(0, cfg.H, 4):
        hs = slice(h0, h0 + 4)
        want_all = ref.based_chunked(q[:, hs], k[:, hs], v[:, hs], chunk=256, dtype=torch.float64)
        e0 = max(e0, max(head_errs(y[:, hs], want_all)))
    n = 1024
    want, _, _ = ref.based_dense(q[:, :, :n], k[:, :, :n], v[:, :, :n])
    e1 = err(y[:, :, :n], want)
    e2 = 0.0
    for h in (0, 9):
        for r0 in (20000, cfg.N - 32):
            rows = torch.arange(r0, r0 + 32)
            e2 = max(e2, ref.rel_err(y[0, h, rows], _rows_fp64(q, k, v, 0, h, rows)))
    phik = ref.taylor_feature_map(k[0, 3].double())
    want_st = torch.cat([phik.T @ v[0, 3].double(), phik.sum(0).unsqueeze(-1)], dim=-1)
    e3 = ref.rel_err(st[0, 3].cpu(), want_st)
    print(f"chunked B1 H16 N65536 all rows worst head err={e0:.3e} prefix err={e1:.3e} rows err={e2:.3e} "
          f"state err={e3:.3e}")
    assert e0 < TOL and e1 < TOL and e2 < TOL and e3 < 1e-2


def test_fp32_inputs_route_to_exact_path():
    K = _kernels()
    q, k, v = rand_qkv(1, 2, 200, 16, 32, seed=3, dtype=torch.float32)
    num = K.chunked_nki_numerator(*to_dev(q, k, v))
    _, want_num, _ = ref.based_dense(q, k, v)
    assert num.dtype == torch.float32
    assert err(num, want_num) < 1e-4


def test_other_head_dims_use_the_parallel_kernel():
    """d = 80 is outside both chunked paths: the parallel kernel computes it, and a state
    (which would have 3321 features) is refused."""
    K = _kernels()
    q, k, v = rand_qkv(1, 2, 150, 80, 16, seed=0, dtype=torch.bfloat16)
    y = K.chunked_based_attn(*to_dev(q, k, v))
    want, _, _ = ref.based_dense(q, k, v)
    assert err(y.float(), want) < 3e-2
    with pytest.raises(RuntimeError):
        K.based_chunked(*to_dev(q, k, v), return_state=True)
