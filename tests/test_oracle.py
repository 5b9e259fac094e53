"""Pins the CPU oracle (oracle/reference.py) before anything is compared against it.

Each restated function is checked against something that does not share its formula:
brute-force Python loops from the definition, closed forms for special inputs, the exact
feature-map identity, a library routine (scaled_dot_product_attention), invariances, and
cross-checks between the dense, phi-form and chunked restatements.  ``test_planted_*``
plant plausible mistakes in copies of the oracle and show that these checks reject them.
"""

import math
import os

import numpy as np
import pytest
import torch
from hypothesis import given, settings, strategies as st

from oracle import reference as ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _inputs(B, H, N, d, dv, seed, dtype=torch.float64, scale_qk=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, N, d, generator=g, dtype=torch.float64) * scale_qk
    k = torch.randn(B, H, N, d, generator=g, dtype=torch.float64) * scale_qk
    v = torch.randn(B, H, N, dv, generator=g, dtype=torch.float64)
    return q.to(dtype), k.to(dtype), v.to(dtype)


# ---------------------------------------------------------------- dense BASED vs brute force

@pytest.mark.parametrize("shape", [(1, 1, 1, 1, 1), (1, 2, 5, 4, 3), (2, 1, 8, 3, 6), (1, 1, 7, 16, 2)])
def test_dense_matches_loops(shape):
    q, k, v = _inputs(*shape, seed=1)
    want = ref.based_loops(q, k, v)
    y, _, _ = ref.based_dense(q, k, v)
    assert np.abs(y.numpy() - want).max() < 1e-12
    # the reference restatement itself, run in fp64
    assert np.abs(ref.ref_based_attn(q, k, v).numpy() - want).max() < 1e-12


@settings(max_examples=25, deadline=None)
@given(B=st.integers(1, 2), H=st.integers(1, 2), N=st.integers(1, 9), d=st.integers(1, 6),
       dv=st.integers(1, 5), seed=st.integers(0, 10_000))
def test_dense_matches_loops_hypothesis(B, H, N, d, dv, seed):
    q, k, v = _inputs(B, H, N, d, dv, seed)
    want = ref.based_loops(q, k, v)
    y, num, den = ref.based_dense(q, k, v)
    assert np.abs(y.numpy() - want).max() < 1e-11
    assert torch.allclose(num / (den + ref.EPS).unsqueeze(-1), y, atol=0, rtol=1e-14)


# ---------------------------------------------------------------- closed forms

def test_zero_queries_reduce_to_cumulative_mean():
    # q = 0  =>  s = 0, p = 1  =>  y_t = cumsum(v)_t / (t + 1 + eps)
    _, k, v = _inputs(1, 2, 33, 8, 5, seed=2)
    q = torch.zeros_like(k)
    y, _, den = ref.based_dense(q, k, v)
    t = torch.arange(1, 34, dtype=torch.float64).view(1, 1, -1, 1)
    want = v.cumsum(-2) / (t + ref.EPS)
    assert torch.allclose(y, want, rtol=1e-14, atol=0)
    assert torch.equal(den, t.squeeze(-1).expand_as(den))


def test_first_row_closed_form():
    # row 0 sees only key 0: y_0 = v_0 p / (p + eps), p = 1 + s + s^2/2
    q, k, v = _inputs(2, 3, 4, 16, 7, seed=3, scale_qk=2.0)
    y, _, _ = ref.based_dense(q, k, v)
    s = (q[..., 0, :] * k[..., 0, :]).sum(-1) / 4.0
    p = 1 + s + 0.5 * s * s
    assert torch.allclose(y[..., 0, :], v[..., 0, :] * (p / (p + ref.EPS)).unsqueeze(-1), rtol=1e-14)


def test_constant_values():
    # v = c  =>  y_t = c * sum p / (sum p + eps)
    q, k, _ = _inputs(1, 2, 21, 4, 1, seed=4, scale_qk=1.5)
    v = torch.full((1, 2, 21, 3), 0.75, dtype=torch.float64)
    y, _, den = ref.based_dense(q, k, v)
    want = 0.75 * den / (den + ref.EPS)
    assert torch.allclose(y, want.unsqueeze(-1).expand_as(y), rtol=1e-13)


def test_causal_prefix_invariance():
    q, k, v = _inputs(1, 2, 40, 8, 4, seed=5)
    y_full, _, _ = ref.based_dense(q, k, v)
    y_pre, _, _ = ref.based_dense(q[:, :, :17], k[:, :, :17], v[:, :, :17])
    assert torch.allclose(y_full[:, :, :17], y_pre, rtol=1e-14, atol=0)


def test_head_permutation_equivariance():
    q, k, v = _inputs(2, 3, 12, 4, 4, seed=6)
    y, _, _ = ref.based_dense(q, k, v)
    perm = torch.tensor([2, 0, 1])
    yp, _, _ = ref.based_dense(q[:, perm], k[:, perm], v[:, perm])
    assert torch.equal(yp, y[:, perm])


# ---------------------------------------------------------------- feature map

@pytest.mark.parametrize("d,F", [(1, 3), (4, 15), (16, 153), (64, 2145)])
def test_feature_dim(d, F):
    assert ref.feature_dim(d) == F
    assert ref.taylor_feature_map(torch.zeros(2, d)).shape == (2, F)


def test_feature_map_element_order():
    x = torch.tensor([[2.0, 3.0, 5.0]], dtype=torch.float64)
    d = 3
    rd, rrd, r2 = math.sqrt(d), d ** 0.25, math.sqrt(2.0)
    want = [1.0, 2 / rrd, 3 / rrd, 5 / rrd, 4 / (rd * r2), 9 / (rd * r2), 25 / (rd * r2),
            6 / rd, 10 / rd, 15 / rd]   # diagonal, then (0,1), (0,2), (1,2)
    assert torch.allclose(ref.taylor_feature_map(x)[0], torch.tensor(want, dtype=torch.float64), rtol=1e-15)


@pytest.mark.parametrize("d", [1, 4, 16, 64])
def test_feature_map_identity(d):
    q, k, _ = _inputs(1, 1, 9, d, 1, seed=7, scale_qk=1.3)
    lhs = ref.taylor_feature_map(q) @ ref.taylor_feature_map(k).transpose(-2, -1)
    s = q @ k.transpose(-2, -1) / math.sqrt(d)
    assert torch.allclose(lhs, 1 + s + 0.5 * s * s, rtol=1e-12, atol=1e-12)


def test_phi_pow_scale_matches_feature_map():
    x, _, _ = _inputs(1, 1, 11, 16, 1, seed=8)
    assert torch.allclose(ref.phi_pow_scale(x, 1 / 4.0), ref.taylor_feature_map(x), rtol=1e-14, atol=1e-15)


# ---------------------------------------------------------------- phi-form and chunked

def test_phi_forms_agree_with_dense():
    q, k, v = _inputs(1, 2, 50, 16, 8, seed=9)
    y, num, _ = ref.based_dense(q, k, v)
    y32, num32, _ = ref.based_dense(q.float(), k.float(), v.float(), dtype=torch.float64)
    assert torch.allclose(ref.ref_based_attn_phi(q.float(), k.float(), v.float()).double(), y32, rtol=1e-4, atol=1e-5)
    assert torch.allclose(ref.ref_based_numerator(q.float(), k.float(), v.float()).double(), num32,
                          rtol=1e-4, atol=1e-4)
    # the phi-form computes in fp32 even for fp64 inputs (.float() at :57-58) and casts back
    y_phi = ref.ref_based_attn_phi(q, k, v)
    assert y_phi.dtype == torch.float64
    assert ref.rel_err(y_phi, y) < 1e-5


@pytest.mark.parametrize("chunk", [1, 3, 16, 64, 1000])
def test_chunked_matches_dense(chunk):
    q, k, v = _inputs(2, 1, 70, 4, 5, seed=10, scale_qk=1.2)
    y, num, _ = ref.based_dense(q, k, v)
    yc = ref.based_chunked(q, k, v, chunk=chunk, dtype=torch.float64)
    nc = ref.based_chunked(q, k, v, chunk=chunk, dtype=torch.float64, normalize=False)
    assert torch.allclose(yc, y, rtol=1e-11, atol=1e-12)
    assert torch.allclose(nc, num, rtol=1e-11, atol=1e-11)


def test_chunked_final_state_closed_form():
    q, k, v = _inputs(1, 2, 37, 4, 3, seed=11)
    _, S, z = ref.based_chunked(q, k, v, chunk=8, dtype=torch.float64, return_state=True)
    phik = ref.taylor_feature_map(k)
    assert torch.allclose(S, phik.transpose(-2, -1) @ v, rtol=1e-12, atol=1e-12)
    assert torch.allclose(z, phik.sum(-2), rtol=1e-12, atol=1e-12)
    assert torch.allclose(z[..., 0], torch.full_like(z[..., 0], 37.0))


def _identity_loops(q, k, v):
    """Causal identity-map numerator from the definition, scalar fp64 loops:
    out[t] = sum_{u <= t} (q_t . k_u / sqrt(d)) v_u."""
    qa, ka, va = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    b, h, t, d = qa.shape
    dv = va.shape[-1]
    out = np.zeros((b, h, t, dv))
    for bi in range(b):
        for hi in range(h):
            for ti in range(t):
                for ui in range(ti + 1):
                    s = sum(qa[bi, hi, ti, e] * ka[bi, hi, ui, e] for e in range(d)) / math.sqrt(d)
                    for e in range(dv):
                        out[bi, hi, ti, e] += s * va[bi, hi, ui, e]
    return out


@pytest.mark.parametrize("shape", [(1, 1, 6, 4, 2), (2, 3, 9, 5, 3), (1, 2, 13, 16, 7)])
def test_identity_numerator_brute_force(shape):
    """ref_identity_numerator against scalar loops (odd d makes 1/sqrt(d) irrational; a
    missing mask, a transposed product or the scale on both q and k fails this)."""
    q, k, v = _inputs(*shape, seed=12)
    got = ref.ref_identity_numerator(q, k, v).numpy()
    want = _identity_loops(q, k, v)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_identity_planted_mistakes_are_caught():
    q, k, v = _inputs(1, 2, 9, 5, 3, seed=13)
    want = _identity_loops(q, k, v)
    d = q.shape[-1]
    mask = torch.tril(torch.ones(9, 9, dtype=q.dtype))
    wrong = [
        (q / math.sqrt(d)) @ k.transpose(-2, -1) @ v,                                   # no causal mask
        ((q / d) @ k.transpose(-2, -1) * mask) @ v,                                     # 1/d instead of 1/sqrt(d)
        ((q / math.sqrt(d)) @ k.transpose(-2, -1) * torch.tril(mask, -1)) @ v,          # strict mask
        (((q / math.sqrt(d)) @ k.transpose(-2, -1)).transpose(-2, -1) * mask) @ v,     # transposed scores
    ]
    for w in wrong:
        assert not np.allclose(w.numpy(), want, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------- sliding window

@pytest.mark.parametrize("w", [1, 2, 5, 64])
def test_sliding_matches_loops(w):
    q, k, v = _inputs(1, 2, 9, 4, 3, seed=13)
    want = ref.sliding_loops(q, k, v, w)
    assert np.abs(ref.sliding_dense(q, k, v, window_size=w).numpy() - want).max() < 1e-12
    # the restated reference computes in fp32 (.float() at :40) and casts back
    assert np.abs(ref.ref_sliding_window_attn(q, k, v, window_size=w).numpy() - want).max() < 1e-6


def test_sliding_full_window_is_causal_sdpa():
    q, k, v = _inputs(1, 2, 40, 8, 8, seed=14)
    want = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert torch.allclose(ref.sliding_dense(q, k, v, window_size=40), want, rtol=1e-12, atol=1e-12)
    assert torch.allclose(ref.sliding_dense(q, k, v, window_size=4096), want, rtol=1e-12, atol=1e-12)


def test_sliding_window_one_is_identity():
    q, k, v = _inputs(1, 2, 17, 8, 5, seed=15)
    assert torch.equal(ref.sliding_dense(q, k, v, window_size=1), v)


def test_sliding_rows_are_convex_combinations():
    q, k, _ = _inputs(1, 2, 30, 8, 1, seed=16, scale_qk=3.0)
    v = torch.ones(1, 2, 30, 4, dtype=torch.float64)
    assert torch.allclose(ref.sliding_dense(q, k, v, window_size=7), v, rtol=1e-14)


@pytest.mark.parametrize("w", [1, 3, 64])
def test_layer_is_sum_of_branches_with_own_projections(w):
    """Full BASED layer (kernels/nki_attention_sliding.py:4-5) against brute force: the linear
    branch on (q, k, v) and the softmax branch on (q_sw, k_sw, v), with d_sw != d."""
    q, k, v = _inputs(1, 2, 9, 4, 3, seed=21)
    q_sw, k_sw, _ = _inputs(1, 2, 9, 6, 3, seed=22)
    want = ref.based_loops(q, k, v) + ref.sliding_loops(q_sw, k_sw, v, w)
    got = ref.based_layer_dense(q, k, v, window_size=w, q_sw=q_sw, k_sw=k_sw)
    assert np.abs(got.numpy() - want).max() < 1e-12
    # the restated reference computes each branch as the reference does (fp32 inside for the
    # softmax branch) and sums them
    got32 = ref.ref_based_layer(q, k, v, window_size=w, q_sw=q_sw, k_sw=k_sw)
    assert np.abs(got32.numpy() - want).max() < 1e-6
    # default projections: both branches on q, k
    want_same = ref.based_loops(q, k, v) + ref.sliding_loops(q, k, v, w)
    assert np.abs(ref.based_layer_dense(q, k, v, window_size=w).numpy() - want_same).max() < 1e-12


def test_sliding_banded_matches_dense():
    q, k, v = _inputs(1, 2, 300, 8, 4, seed=17)
    for w in (1, 13, 64, 300):
        assert torch.allclose(ref.sliding_banded(q, k, v, window_size=w, dtype=torch.float64, block=37),
                              ref.sliding_dense(q, k, v, window_size=w), rtol=1e-12, atol=1e-13)


def test_reference_dtype_is_kept():
    q, k, v = ref.make_inputs(1, 1, 8, 16, 4, torch.bfloat16, 0)
    assert ref.ref_based_attn(q, k, v).dtype == torch.bfloat16
    assert ref.ref_sliding_window_attn(q, k, v, 4).dtype == torch.bfloat16
    assert ref.ref_based_attn_phi(q, k, v).dtype == torch.bfloat16


# ---------------------------------------------------------------- planted mistakes

def _planted_variants():
    def dropped_square(q, k, v, eps=ref.EPS):
        s = q @ k.transpose(-2, -1) / math.sqrt(q.shape[-1])
        p = (1 + s) * torch.tril(torch.ones(s.shape[-2:], dtype=s.dtype))
        return (p @ v) / (p.sum(-1, keepdim=True) + eps)

    def strict_mask(q, k, v, eps=ref.EPS):
        s = q @ k.transpose(-2, -1) / math.sqrt(q.shape[-1])
        p = (1 + s + 0.5 * s * s) * torch.tril(torch.ones(s.shape[-2:], dtype=s.dtype), -1)
        return (p @ v) / (p.sum(-1, keepdim=True) + eps)

    def transposed_scores(q, k, v, eps=ref.EPS):
        s = k @ q.transpose(-2, -1) / math.sqrt(q.shape[-1])
        p = (1 + s + 0.5 * s * s) * torch.tril(torch.ones(s.shape[-2:], dtype=s.dtype))
        return (p @ v) / (p.sum(-1, keepdim=True) + eps)

    def scale_on_both(q, k, v, eps=ref.EPS):
        c = 1 / math.sqrt(q.shape[-1])
        s = (q * c) @ (k * c).transpose(-2, -1)
        p = (1 + s + 0.5 * s * s) * torch.tril(torch.ones(s.shape[-2:], dtype=s.dtype))
        return (p @ v) / (p.sum(-1, keepdim=True) + eps)

    def eps_in_numerator(q, k, v, eps=ref.EPS):
        s = q @ k.transpose(-2, -1) / math.sqrt(q.shape[-1])
        p = (1 + s + 0.5 * s * s) * torch.tril(torch.ones(s.shape[-2:], dtype=s.dtype))
        return (p @ v + 1e-3) / (p.sum(-1, keepdim=True))

    return [dropped_square, strict_mask, transposed_scores, scale_on_both, eps_in_numerator]


@pytest.mark.parametrize("variant", _planted_variants(), ids=lambda f: f.__name__)
def test_planted_based_mistakes_are_caught(variant):
    q, k, v = _inputs(1, 2, 6, 4, 3, seed=18, scale_qk=1.5)
    want = ref.based_loops(q, k, v)
    assert np.abs(variant(q, k, v).numpy() - want).max() > 1e-6


def test_planted_sliding_off_by_one_is_caught():
    q, k, v = _inputs(1, 1, 12, 4, 3, seed=19)
    want = ref.sliding_loops(q, k, v, 3)
    wrong = ref.sliding_dense(q, k, v, window_size=4)   # window one too wide
    assert np.abs(wrong.numpy() - want).max() > 1e-6


def test_planted_chunk_state_order_is_caught():
    # updating the state before the inter-chunk read double-counts the chunk
    q, k, v = _inputs(1, 1, 16, 4, 2, seed=20)
    qf, kf = ref.taylor_feature_map(q[0, 0]), ref.taylor_feature_map(k[0, 0])
    S = torch.zeros(qf.shape[-1], 2, dtype=torch.float64)
    outs = []
    for c0 in range(0, 16, 4):
        qc, kc, vc = qf[c0:c0 + 4], kf[c0:c0 + 4], v[0, 0, c0:c0 + 4]
        S = S + kc.T @ vc
        outs.append(qc @ S + torch.tril(qc @ kc.T) @ vc)
    wrong = torch.cat(outs)
    _, num, _ = ref.based_dense(q, k, v)
    assert (wrong - num[0, 0]).abs().max() > 1e-6


# ---------------------------------------------------------------- golden fixtures

def _load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as f:
        return {key: f[key] for key in f.files}


@pytest.mark.parametrize("name", ["based_b1h2n67d16dv64", "based_b1h1n130d16dv16", "based_b1h2n129d4dv8",
                                  "based_b1h2n67d16dv64_unscaled"])
def test_golden_based(name):
    g = _load(name)
    q, k, v = (torch.from_numpy(g[x]) for x in "qkv")
    # inputs are bf16-representable
    assert torch.equal(q.to(torch.bfloat16).float(), q)
    y, num, den = ref.based_dense(q, k, v)
    assert np.abs(y.numpy() - g["y"]).max() < 1e-12
    assert np.abs(den.numpy() - g["den"]).max() < 1e-9
    # brute force on a prefix (causal prefix invariance makes the prefix self-contained)
    n = 6
    want = ref.based_loops(q[:, :, :n], k[:, :, :n], v[:, :, :n])
    assert np.abs(g["y"][:, :, :n] - want).max() < 1e-12


@pytest.mark.parametrize("name", ["sliding_b1h2n131d64w1", "sliding_b1h2n131d64w17", "sliding_b1h2n131d64w64"])
def test_golden_sliding(name):
    g = _load(name)
    q, k, v = (torch.from_numpy(g[x]) for x in "qkv")
    w = int(g["window"])
    y = ref.sliding_dense(q, k, v, window_size=w)
    assert np.abs(y.numpy() - g["y"]).max() < 1e-12
    n = 5
    want = ref.sliding_loops(q[:, :1, :n], k[:, :1, :n], v[:, :1, :n], w)
    assert np.abs(g["y"][:, :1, :n] - want).max() < 1e-12


@pytest.mark.parametrize("name", ["phi_d4", "phi_d16"])
def test_golden_feature_map(name):
    g = _load(name)
    x = torch.from_numpy(g["x"]).double()
    assert np.abs(ref.taylor_feature_map(x).numpy() - g["phi"]).max() < 1e-14


def test_inputs_are_seeded_and_ordered():
    a = ref.make_inputs(1, 2, 8, 4, 3, torch.float32, 5, prescale=False)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 2, 8, 4, generator=g)
    k = torch.randn(1, 2, 8, 4, generator=g)
    v = torch.randn(1, 2, 8, 3, generator=g)
    assert torch.equal(a[0], q) and torch.equal(a[1], k) and torch.equal(a[2], v)
    b = ref.make_inputs(1, 2, 8, 4, 3, torch.float32, 5, prescale=True)
    assert torch.allclose(b[0], q / 2.0) and torch.allclose(b[1], k / 2.0) and torch.equal(b[2], v)
