"""State export and import on the segment-state chunked shapes (bf16 d != 16 or dv > 64, fp32
inputs): ``based_chunked(..., return_state=True / state_in=...)`` through
la_based_chunked_fwd_num_den, la_taylor_feature_map and fp32 GEMMs.

Checks: the exported state against its closed form sum_u phi(k_u) [v_u | 1] (fp64 on the same
rounded inputs), a sequence cut into pieces that pass the state along against dense BASED over
the whole sequence (the oracle), prefill -> decode -> continue on a d = 64 state, the
numerator/denominator entry point against the normalised one, and at B2 H16 N8192 d64 a cut
sequence against the uncut call plus fp64 spot rows.  Bars: 2e-2 for bf16 inputs, 1e-4 for
fp32 (max |y - y_ref| / rms(y_ref)); states 1e-2 (bf16) and 1e-4 (fp32) relative to their rms
(the largest state entries, the constant feature's row sum_u v_u and the count, sit far above
the rms, so their fp32 rounding dominates the max).
"""

import math

import pytest
import torch

from oracle import reference as ref
from tests.helpers import err, rand_qkv, rows_fp64, to_dev

pytestmark = pytest.mark.gpu

BARS = {torch.bfloat16: 2e-2, torch.float32: 1e-4}
STATE_BARS = {torch.bfloat16: 1e-2, torch.float32: 1e-4}
CASES = [(torch.bfloat16, 64, 64), (torch.bfloat16, 32, 128), (torch.bfloat16, 16, 100),
         (torch.float32, 16, 64), (torch.float32, 64, 48)]


def _kernels():
    import kernels
    return kernels


def _closed_form(k, v, scale=None):
    d = k.shape[-1]
    a = 1.0 if scale is None else math.sqrt(scale * math.sqrt(d))
    phik = ref.taylor_feature_map(k.double() * a)
    return torch.cat([phik.transpose(-2, -1) @ v.double(), phik.sum(-2).unsqueeze(-1)], dim=-1)


@pytest.mark.parametrize("dt,d,dv", CASES)
def test_state_closed_form(dt, d, dv):
    K = _kernels()
    q, k, v = rand_qkv(1, 3, 1300, d, dv, seed=d + dv, dtype=dt, scale_qk=0.6)
    y, st = K.based_chunked(*to_dev(q, k, v), out_dtype=torch.float32, return_state=True)
    want_st = _closed_form(k, v)
    es = ref.rel_err(st.cpu(), want_st)
    want, _, _ = ref.based_dense(q, k, v)
    e = err(y, want)
    print(f"{dt} d={d} dv={dv} state err={es:.3e} out err={e:.3e}")
    assert st.shape == (1, 3, K.feature_dim(d), dv + 1)
    assert es < STATE_BARS[dt] and e < BARS[dt]


@pytest.mark.parametrize("normalize", [True, False])
@pytest.mark.parametrize("dt,d,dv", CASES)
def test_pieces_match_dense(dt, d, dv, normalize):
    """The sequence in three calls (the middle one ragged, one shorter than a segment), each
    continuing the previous state, against dense BASED over the whole sequence; the last
    state against the closed form over all tokens."""
    K = _kernels()
    B, H, cuts = 2, 2, [0, 700, 1013, 2100]
    q, k, v = rand_qkv(B, H, cuts[-1], d, dv, seed=7 * d + dv, dtype=dt, scale_qk=0.5)
    qd, kd, vd = to_dev(q, k, v)
    ys, st = [], None
    for a, b in zip(cuts[:-1], cuts[1:]):
        y, st = K.based_chunked(qd[:, :, a:b], kd[:, :, a:b], vd[:, :, a:b], out_dtype=torch.float32,
                                normalize=normalize, return_state=True, state_in=st)
        ys.append(y)
    y = torch.cat(ys, dim=2)
    want, want_num, _ = ref.based_dense(q, k, v)
    e = err(y, want if normalize else want_num)
    es = ref.rel_err(st.cpu(), _closed_form(k, v))
    print(f"{dt} d={d} dv={dv} normalize={normalize} pieces err={e:.3e} state err={es:.3e}")
    assert e < BARS[dt] and es < STATE_BARS[dt]


def test_scale_with_state():
    """A scale other than 1/sqrt(d): the state is phi(a k) with a = (scale^2 d)^(1/4), and the
    continuation applies it to phi(a q)."""
    K = _kernels()
    scale = 0.05
    q, k, v = rand_qkv(1, 2, 1500, 64, 64, seed=3, dtype=torch.bfloat16)
    qd, kd, vd = to_dev(q, k, v)
    _, st = K.based_chunked(qd[:, :, :600], kd[:, :, :600], vd[:, :, :600], scale=scale, return_state=True,
                            out_dtype=torch.float32)
    y2 = K.based_chunked(qd[:, :, 600:], kd[:, :, 600:], vd[:, :, 600:], scale=scale, state_in=st,
                         out_dtype=torch.float32)
    want, _, _ = ref.based_dense(q, k, v, scale=scale)
    e = err(y2, want[:, :, 600:])
    es = ref.rel_err(st.cpu(), _closed_form(k[:, :, :600], v[:, :, :600], scale=scale))
    print(f"scale={scale} continuation err={e:.3e} state err={es:.3e}")
    assert e < 2e-2 and es < 1e-2


def test_empty_pieces():
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(1, 2, 300, 64, 32, seed=1, dtype=torch.bfloat16))
    _, st = K.based_chunked(q, k, v, return_state=True)
    e = q[:, :, :0]
    y0, st0 = K.based_chunked(e, k[:, :, :0], v[:, :, :0], return_state=True)
    assert y0.shape == (1, 2, 0, 32) and float(st0.abs().max()) == 0.0
    y1, st1 = K.based_chunked(e, k[:, :, :0], v[:, :, :0], return_state=True, state_in=st)
    assert y1.shape == (1, 2, 0, 32) and torch.equal(st1, st)


def test_num_den_entry_point():
    """la_based_chunked_fwd_num_den: num / (den + eps) equals la_based_chunked_fwd's output and
    den equals the dense row sums of p, on both chunked paths."""
    K = _kernels()
    from kernels import _lib
    L = _lib.lib()
    for dt, d, dv in [(torch.bfloat16, 16, 64), (torch.bfloat16, 64, 64), (torch.float32, 16, 40)]:
        q, k, v = rand_qkv(1, 2, 1100, d, dv, seed=d * dv, dtype=dt, scale_qk=0.5)
        qd, kd, vd = to_dev(q, k, v)
        B, H, N = q.shape[:3]
        code = _lib.dtype_code(dt)
        wsb = int(L.la_based_chunked_workspace_bytes_dt(B, H, N, d, dv, 64, code))
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
        num = torch.empty(B, H, N, dv, device="cuda")
        den = torch.empty(B, H, N, device="cuda")
        rc = L.la_based_chunked_fwd_num_den(_lib.ptr(qd), _lib.ptr(kd), _lib.ptr(vd), code, _lib.ptr(num),
                                            _lib.ptr(den), B, H, N, d, dv, 64, 1.0 / math.sqrt(d), _lib.ptr(ws),
                                            wsb, 0)
        assert rc == 0
        torch.cuda.synchronize()
        want, want_num, _ = ref.based_dense(q, k, v)
        s = (q.double() / math.sqrt(d)) @ k.double().transpose(-2, -1)
        p = (1 + s + 0.5 * s * s).tril()
        want_den = p.sum(-1)
        en, ed = err(num, want_num), ref.rel_err(den.cpu(), want_den)
        ey = err(num / (den + 1e-6).unsqueeze(-1), want)
        print(f"{dt} d={d} dv={dv} num err={en:.3e} den err={ed:.3e} y err={ey:.3e}")
        bar = BARS[dt]
        assert en < bar and ed < bar / 10 and ey < bar


def test_prefill_decode_continue_d64():
    """Prefill with state export, decode steps on the exported d = 64 state, then a chunked
    continuation from the decoded state, against dense BASED over the whole sequence."""
    K = _kernels()
    n0, nd, n2 = 700, 5, 400
    T = n0 + nd + n2
    q, k, v = rand_qkv(2, 2, T, 64, 64, seed=21, dtype=torch.bfloat16, scale_qk=0.6)
    qd, kd, vd = to_dev(q, k, v)
    y0, st = K.based_chunked(qd[:, :, :n0], kd[:, :, :n0], vd[:, :, :n0], out_dtype=torch.float32,
                             return_state=True)
    st = st.contiguous()
    yd = []
    for t in range(n0, n0 + nd):
        yd.append(K.based_decode_step(qd[:, :, t].float(), kd[:, :, t].float(), vd[:, :, t].float(), st))
    y2 = K.based_chunked(qd[:, :, n0 + nd:], kd[:, :, n0 + nd:], vd[:, :, n0 + nd:], out_dtype=torch.float32,
                         state_in=st)
    y = torch.cat([y0, torch.stack(yd, dim=2), y2], dim=2)
    want, _, _ = ref.based_dense(q, k, v)
    e = err(y, want)
    print(f"prefill/decode/continue d64 err={e:.3e}")
    assert e < 2e-2


def test_b2h16n8192_d64_cut():
    """B2 H16 N8192 d = 64 (the reference's chunked head dim) cut at 3000 and 5000: the pieces
    against the uncut call, fp64 rows of three heads after each cut and the final state of two
    heads against the closed form."""
    K = _kernels()
    q, k, v = ref.make_inputs(2, 16, 8192, 64, 64, torch.bfloat16, seed=40, prescale=False)
    qd, kd, vd = to_dev(q, k, v)
    full = K.based_chunked(qd, kd, vd, out_dtype=torch.float32).cpu()
    ys, st = [], None
    for a, b in [(0, 3000), (3000, 5000), (5000, 8192)]:
        y, st = K.based_chunked(qd[:, :, a:b], kd[:, :, a:b], vd[:, :, a:b], out_dtype=torch.float32,
                                return_state=True, state_in=st)
        ys.append(y.cpu())
    y = torch.cat(ys, dim=2)
    del ys
    e0 = ref.rel_err(y, full)
    e1 = 0.0
    for b, h in [(0, 0), (0, 9), (1, 15)]:
        for r0 in (3000, 5000, 8192 - 32):
            rows = torch.arange(r0, r0 + 32)
            e1 = max(e1, ref.rel_err(y[b, h, rows], rows_fp64(q, k, v, b, h, rows)))
    es = max(ref.rel_err(st[b, h].cpu(), _closed_form(k[b, h], v[b, h])) for b, h in [(0, 3), (1, 12)])
    print(f"B2 H16 N8192 d64 cut vs uncut={e0:.3e} rows={e1:.3e} state={es:.3e}")
    assert e0 < 2e-2 and e1 < 2e-2 and es < 1e-2
