"""Numeric range of the bf16 kernels: inputs far from N(0, 1) against the fp64 oracle.

The bf16 kernels run their products on fp16 MFMAs (V, the rounded polynomial, the features and
the chunked state), whose range is 2^-14 .. 65504 against bf16's 2^-126 .. 3.4e38.  These cases
hold each kernel to the bf16 bar (max|y - y_ref| / rms(y_ref) < 2e-2 per head, fp32 output) for
bf16 inputs of any magnitude the reference's own bf16 arithmetic handles
(kernels/pytorch_attention.py:35-41): V scaled by 1e5 and 1e-6, heads of different scales in one
call, blocks of one head on both sides of the kernels' scale steps, scores s = q.k/sqrt(d) up to
about 300, a mean-biased V over 65536 tokens (its sums grow linearly with N), the long-context
configuration without pre-scaling, and a continuation from a state with a large sum of v.
The fp32 inputs that run as three bf16 terms per operand are held to the fp32 bar for V scaled
by 1e30 and 1e-30 and for large scores, and the sliding-window softmax (resident and streaming
kernels) to the bf16 bar for the same V scales and scores of several hundred.
"""

import pytest
import torch

from oracle import reference as ref
from tests.helpers import err, head_errs, rand_qkv, rows_fp64, to_dev

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _kernels():
    import kernels
    return kernels


def _scaled(B, H, N, d, dv, seed, vscale=1.0, qk=0.5, vbias=0.0):
    q, k, v = rand_qkv(B, H, N, d, dv, seed=seed, dtype=torch.float32, scale_qk=qk)
    v = v * torch.as_tensor(vscale, dtype=torch.float32) + vbias
    return q.bfloat16(), k.bfloat16(), v.bfloat16()


def _run(path, q, k, v, normalize=True):
    K = _kernels()
    qd, kd, vd = to_dev(q, k, v)
    if path == "parallel":
        return K.based_parallel(qd, kd, vd, normalize=normalize, out_dtype=torch.float32)
    return K.based_chunked(qd, kd, vd, normalize=normalize, out_dtype=torch.float32)


# (d, dv): the packed parallel kernel (d 16, dv % 8 == 0, dv <= 64), the register-staged one
# (d 32; dv 96) and the chunked kernel's shapes
PAR_SHAPES = [(16, 64), (16, 40), (32, 64), (16, 96)]


@pytest.mark.parametrize("vscale", [1e5, 1e-6, 3e4, 2e-5])
@pytest.mark.parametrize("d,dv", PAR_SHAPES)
def test_parallel_v_scale(vscale, d, dv):
    q, k, v = _scaled(1, 2, 1100, d, dv, seed=11, vscale=vscale)
    want, want_num, _ = ref.based_dense(q, k, v)
    e = max(head_errs(_run("parallel", q, k, v), want))
    en = max(head_errs(_run("parallel", q, k, v, normalize=False), want_num))
    print(f"parallel d={d} dv={dv} v x {vscale:g}: err={e:.3e} num_err={en:.3e}")
    assert e < TOL and en < TOL


@pytest.mark.parametrize("vscale", [1e5, 1e-6, 3e4])
@pytest.mark.parametrize("dv", [64, 24])
def test_chunked_v_scale(vscale, dv):
    q, k, v = _scaled(1, 2, 3000, 16, dv, seed=12, vscale=vscale)
    want, want_num, _ = ref.based_dense(q, k, v)
    e = max(head_errs(_run("chunked", q, k, v), want))
    en = max(head_errs(_run("chunked", q, k, v, normalize=False), want_num))
    print(f"chunked dv={dv} v x {vscale:g}: err={e:.3e} num_err={en:.3e}")
    assert e < TOL and en < TOL


@pytest.mark.parametrize("path,d,dv", [("parallel", 16, 64), ("parallel", 32, 64), ("chunked", 16, 64)])
def test_heads_of_different_scales(path, d, dv):
    """One call, four heads at V scales 1e5, 1, 1e-6 and 1e-3: each head on its own scale."""
    q, k, v = _scaled(1, 4, 1500, d, dv, seed=13, vscale=torch.tensor([1e5, 1.0, 1e-6, 1e-3]).view(1, 4, 1, 1))
    want, _, _ = ref.based_dense(q, k, v)
    errs = head_errs(_run(path, q, k, v), want)
    print(f"{path} d={d} dv={dv} per-head errs " + " ".join(f"{x:.2e}" for x in errs))
    assert max(errs) < TOL


@pytest.mark.parametrize("path,d,dv", [("parallel", 16, 64), ("parallel", 16, 96), ("chunked", 16, 64)])
def test_scale_steps_within_a_head(path, d, dv):
    """V magnitudes that put the 64-key blocks (and 128-token chunks) of one head on different
    sides of the kernels' power-of-two scale steps: |v| near 128, and a head whose first 300
    tokens are 1e6 times smaller than the rest."""
    q, k, v = _scaled(1, 2, 2600, d, dv, seed=14, vscale=40.0)
    t = torch.ones(1, 2, 2600, 1)
    t[:, 1, :300] = 1e-6
    v2 = (v.float() * t).bfloat16()
    for vv in (v, v2):
        want, _, _ = ref.based_dense(q, k, vv)
        errs = head_errs(_run(path, q, k, vv), want)
        print(f"{path} d={d} dv={dv} errs " + " ".join(f"{x:.2e}" for x in errs))
        assert max(errs) < TOL


@pytest.mark.parametrize("path,d,dv", [("parallel", 16, 64), ("parallel", 32, 64), ("parallel", 16, 96),
                                       ("chunked", 16, 64)])
def test_large_scores(path, d, dv):
    """q, k ~ N(0, 7.5^2): typical |s| = |q.k|/sqrt(d) around 60 and the largest near 300, where
    p = 1 + s + s^2/2 reaches 4.5e4."""
    q, k, v = _scaled(1, 2, 1200, d, dv, seed=15, qk=7.5)
    s = (q[0, 0].double() @ k[0, 0].double().T) / d ** 0.5
    smax = s.tril().abs().max().item()
    want, _, _ = ref.based_dense(q, k, v)
    e = max(head_errs(_run(path, q, k, v), want))
    print(f"{path} d={d} dv={dv} max|s|={smax:.0f} err={e:.3e}")
    assert smax > 250
    assert e < TOL


def _long_checks(y, q, k, v, heads, st=None, n=1024):
    """Prefix rows against the dense oracle (causal prefix invariance), spot rows against fp64
    over all earlier keys, the exported state against its closed form."""
    y = y.cpu()
    want, _, _ = ref.based_dense(q[:, heads, :n], k[:, heads, :n], v[:, heads, :n])
    e1 = max(head_errs(y[:, heads, :n], want))
    e2 = 0.0
    N = q.shape[2]
    for h in heads:
        for r0 in (N // 3, N - 32):
            rows = torch.arange(r0, r0 + 32)
            e2 = max(e2, ref.rel_err(y[0, h, rows], rows_fp64(q, k, v, 0, h, rows)))
    e3 = 0.0
    if st is not None:
        h = heads[0]
        phik = ref.taylor_feature_map(k[0, h].double())
        want_st = torch.cat([phik.T @ v[0, h].double(), phik.sum(0).unsqueeze(-1)], dim=-1)
        e3 = ref.rel_err(st[0, h].cpu(), want_st)
    return e1, e2, e3


def test_biased_v_b1h4n65536():
    """v = randn + 1 over 65536 tokens: sum v and every sum phi_f(k) v grow linearly with N."""
    K = _kernels()
    q, k, v = _scaled(1, 4, 65536, 16, 64, seed=16, qk=1.0, vbias=1.0)
    y, st = K.based_chunked(*to_dev(q, k, v), out_dtype=torch.float32, return_state=True)
    e1, e2, e3 = _long_checks(y, q, k, v, [0, 3], st)
    print(f"biased v N65536: prefix err={e1:.3e} rows err={e2:.3e} state err={e3:.3e}")
    assert e1 < TOL and e2 < TOL and e3 < 1e-2


def test_chunked_b1h16n65536_unscaled():
    """The long-context configuration without dividing q and k by sqrt(d)."""
    K = _kernels()
    cfg = ref.CONFIGS["chunked_bf16_b1h16n65536"]
    q, k, v = ref.config_inputs(cfg, prescale=False)
    y, st = K.based_chunked(*to_dev(q, k, v), chunk_size=cfg.chunk, out_dtype=torch.float32, return_state=True)
    e1, e2, e3 = _long_checks(y, q, k, v, [0, 9], st)
    print(f"B1 H16 N65536 unscaled: prefix err={e1:.3e} rows err={e2:.3e} state err={e3:.3e}")
    assert e1 < TOL and e2 < TOL and e3 < 1e-2


def test_continue_from_large_state():
    """A 60000-token prefill of v = randn + 2 exported as a state (sum v ~ 1.2e5 per column),
    then 2000 more tokens continued from it: rows against fp64 over the whole sequence."""
    K = _kernels()
    q, k, v = _scaled(1, 2, 62000, 16, 64, seed=17, qk=1.0, vbias=2.0)
    qd, kd, vd = to_dev(q, k, v)
    n0 = 60000
    _, st = K.based_chunked(qd[:, :, :n0], kd[:, :, :n0], vd[:, :, :n0], out_dtype=torch.float32, return_state=True)
    assert st[0, 0, 0, :64].abs().max().item() > 1e5
    y2 = K.based_chunked(qd[:, :, n0:], kd[:, :, n0:], vd[:, :, n0:], out_dtype=torch.float32, state_in=st,
                         prev_tokens=n0).cpu()
    e = 0.0
    for h in (0, 1):
        for r0 in (0, 1000, 1968):
            rows = torch.arange(n0 + r0, n0 + r0 + 32)
            e = max(e, ref.rel_err(y2[0, h, r0:r0 + 32], rows_fp64(q, k, v, 0, h, rows)))
    print(f"continuation from a large state: rows err={e:.3e}")
    assert e < TOL


TOL_F32 = 1e-4


@pytest.mark.parametrize("vscale,qk", [(1e30, 1.0), (1e-30, 1.0), (1.0, 8.0)])
@pytest.mark.parametrize("B,H,N", [(1, 3, 777), (2, 64, 1024)])
def test_fp32_three_term_range(vscale, qk, B, H, N):
    """fp32 inputs on the kernels that split every operand into three bf16 terms (the small-grid
    kernel at B1 H3, the tiled one at B2 H64): V scaled by 1e30 and 1e-30 (terms of magnitude
    |v|, |v| 2^-8 and |v| 2^-16, all inside bf16's normal range) and scores up to about 300, at
    the fp32 bar against fp64 on the first and last heads."""
    q, k, v = rand_qkv(B, H, N, 16, 64, seed=N + H, dtype=torch.float32, scale_qk=qk)
    v = v * vscale
    y = _kernels().based_parallel(*to_dev(q, k, v), out_dtype=torch.float32).cpu()
    for bb, hh in ((0, 0), (B - 1, H - 1)):
        sl = (slice(bb, bb + 1), slice(hh, hh + 1))
        want, _, _ = ref.based_dense(q[sl], k[sl], v[sl])
        e = err(y[sl], want)
        print(f"fp32 three-term B{B} H{H} N{N} v x {vscale:g} qk x {qk:g} head ({bb},{hh}): err={e:.3e}")
        assert e < TOL_F32


@pytest.mark.parametrize("vscale,qk", [(1e30, 1.0), (1e-30, 1.0), (1.0, 20.0)])
@pytest.mark.parametrize("W", [64, 200])
def test_sliding_range(vscale, qk, W):
    """bf16 sliding-window softmax (the resident kernel at W = 64, the streaming one at W = 200)
    for V far from 1 (the P.V products run on bf16 MFMAs with P split into hi + lo, so V keeps
    bf16's range) and scores of several hundred (softmax in fp32 against the running maximum):
    fp32 output against fp64 at the bf16 bar."""
    q, k, v = _scaled(1, 2, 1000, 64, 64, seed=W + 7, vscale=vscale, qk=qk)
    K = _kernels()
    y = K.sliding_window_attn(*to_dev(q, k, v), window_size=W, out_dtype=torch.float32)
    want = ref.sliding_dense(q, k, v, window_size=W)
    e = max(head_errs(y, want))
    print(f"sliding W={W} v x {vscale:g} qk x {qk:g}: err={e:.3e}")
    assert torch.isfinite(y).all() and e < TOL


def test_general_zero_key_dims_large_v():
    """Segment-state path (d = 64): keys zero in dims 16..63 over the first 512-token segment, so
    the work-groups of feature groups built from those dims see an all-zero state prefix (stored
    as zeros, whatever scale the slot's other part sets), with V scaled by 1e10: finite outputs
    at the bf16 bar against fp64."""
    q, k, v = _scaled(1, 2, 1500, 64, 64, seed=18, vscale=1e10, qk=0.5)
    k = k.clone()
    k[:, :, :512, 16:] = 0
    want, _, _ = ref.based_dense(q, k, v)
    y = _run("chunked", q, k, v)
    errs = head_errs(y, want)
    print(f"general d64 zero key dims, v x 1e10: errs " + " ".join(f"{x:.2e}" for x in errs))
    assert torch.isfinite(y).all() and max(errs) < TOL


@pytest.mark.parametrize("path,d,kscale", [("parallel", 16, 1e4), ("parallel", 32, 1e4), ("chunked", 16, 100.0),
                                           ("chunked", 64, 30.0)])
def test_unbalanced_q_k(path, d, kscale):
    """q divided and k multiplied by the same factor (the scores are unchanged): the parallel
    kernels at 1e4; the d = 16 chunk recurrence, whose features are fp16 products of
    sqrt(scale) q and sqrt(scale) k, at 100 (max |k| about 450 here, inside its limit of 1024);
    the bf16 segment-state path, whose q-side features are fp16 in units of max |[scale q, 1]|,
    at 30 (the stated range of both)."""
    q, k, v = rand_qkv(1, 2, 700, d, 64, seed=3, dtype=torch.float32)
    q, k, v = (q / kscale).bfloat16(), (k * kscale).bfloat16(), v.bfloat16()
    want, _, _ = ref.based_dense(q, k, v)
    y = _run(path, q, k, v)
    e = max(head_errs(y, want))
    print(f"{path} d={d} q / {kscale:g}, k x {kscale:g}: err={e:.3e}")
    assert torch.isfinite(y).all() and e < TOL


@pytest.mark.parametrize("vscale", [1e-20, 1e-36, 1e30])
@pytest.mark.parametrize("path,d,B,H,N", [("parallel", 16, 1, 2, 1100), ("parallel", 32, 1, 2, 1100),
                                          ("chunked", 16, 1, 2, 3000), ("chunked", 16, 2, 16, 2600),
                                          ("chunked", 64, 1, 2, 1500)])
def test_v_extreme_scales(vscale, path, d, B, H, N):
    """V at 1e-20, 1e-36 (near bf16's smallest normal) and 1e30: the fp16 copies of V and of the
    chunked states carry power-of-two exponents (the d = 16 recurrence's unit no lower than
    2^-126; the segment-state path divides V by the head's 2^floor(log2 max|v|) before its fp16
    prefixes, which sit beside the k-sums), so every path holds the bf16 bar."""
    q, k, v = _scaled(B, H, N, d, 64, seed=19, vscale=vscale)
    sl = (slice(0, 1), slice(0, 1))
    want, _, _ = ref.based_dense(q[sl], k[sl], v[sl])
    y = _run(path, q, k, v)
    e = max(head_errs(y[sl], want))
    print(f"{path} d={d} B{B} H{H} N{N} v x {vscale:g}: err={e:.3e}")
    assert torch.isfinite(y).all() and e < TOL


def test_general_v_tiny_prefix():
    """Segment-state path (d = 64): the first 600 tokens' V 1e-20 times the rest, so the first
    segment's prefix is 1e-20 below the later ones (the head exponent comes from the largest)."""
    q, k, v = _scaled(1, 2, 1500, 64, 64, seed=20)
    t = torch.ones(1, 2, 1500, 1)
    t[:, :, :600] = 1e-20
    v = (v.float() * t).bfloat16()
    want, _, _ = ref.based_dense(q, k, v)
    errs = head_errs(_run("chunked", q, k, v), want)
    print("general d64 tiny-V prefix errs " + " ".join(f"{x:.2e}" for x in errs))
    assert max(errs) < TOL


@pytest.mark.parametrize("vscale", [1e-36, 1e30])
def test_v_extreme_scales_other_paths(vscale):
    """The same V scales on the fp32 segment-state path (d 16 and 64, fp32 bar), the identity
    map, the one-launch layer (bf16 output: max |y - y_ref| / (|y_ref| + rms)) and a decode step
    after a prefill."""
    from tests.helpers import rounded_err
    K = _kernels()
    for d in (16, 64):
        q, k, v = rand_qkv(1, 2, 1500, d, 64, seed=4, dtype=torch.float32, scale_qk=0.5)
        v = v * vscale
        want, _, _ = ref.based_dense(q, k, v)
        e = max(head_errs(K.based_chunked(*to_dev(q, k, v), out_dtype=torch.float32), want))
        print(f"fp32 segment-state d={d} v x {vscale:g}: err={e:.3e}")
        assert e < TOL_F32
    q, k, v = _scaled(1, 2, 1000, 16, 64, seed=5, vscale=vscale)
    y = K.identity_linear_attn(*to_dev(q, k, v), out_dtype=torch.float32)
    e = max(head_errs(y, ref.ref_identity_numerator(q.double(), k.double(), v.double())))
    print(f"identity v x {vscale:g}: err={e:.3e}")
    assert e < 1e-3
    q, k, v = _scaled(2, 4, 2600, 16, 64, seed=6, vscale=vscale)
    g = torch.Generator().manual_seed(7)
    qs = (torch.randn(2, 4, 2600, 16, generator=g) * 0.5).bfloat16()
    ks = (torch.randn(2, 4, 2600, 16, generator=g) * 0.5).bfloat16()
    y = K.based_layer_attn(*to_dev(q, k, v, qs, ks)[:3], window_size=64, q_sw=qs.cuda(), k_sw=ks.cuda())
    want = ref.based_layer_dense(q[:, :1], k[:, :1], v[:, :1], window_size=64, q_sw=qs[:, :1], k_sw=ks[:, :1])
    e = rounded_err(y.float()[:, :1], want)
    print(f"layer v x {vscale:g}: err={e:.3e}")
    assert torch.isfinite(y).all() and e < TOL
    q, k, v = _scaled(1, 2, 301, 16, 64, seed=8, vscale=vscale)
    qd, kd, vd = to_dev(q, k, v)
    _, st = K.based_chunked(qd[:, :, :300], kd[:, :, :300], vd[:, :, :300], out_dtype=torch.float32,
                            return_state=True)
    yd = K.based_decode_step(qd[:, :, 300:], kd[:, :, 300:], vd[:, :, 300:], st).float().cpu()
    want, _, _ = ref.based_dense(q, k, v)
    e = rounded_err(yd[:, :, 0], want[:, :, 300])
    print(f"decode after prefill v x {vscale:g}: err={e:.3e}")
    assert torch.isfinite(yd).all() and e < TOL
