"""CPU oracle for BASED causal linear attention and sliding-window softmax attention.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this module; only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it,
and only to check results (or as the timed CPU baseline), never as the computation that is
shipped.

It restates, line by line, the PyTorch math of the reference repository
(Willy-Chan/trainium-linear-attention) on the CPU:

* ``ref_based_attn``            -- kernels/pytorch_attention.py:27-42 (computes in the input dtype)
* ``taylor_feature_map``        -- benchmarks/chunked_attention_benchmark.py:23-53
* ``ref_based_attn_phi``        -- benchmarks/chunked_attention_benchmark.py:55-65 (the phi-form
                                   ``ref_based_attn`` of that module, fp32 inside, cast back)
* ``ref_based_numerator``       -- benchmarks/chunked_attention_benchmark.py:68-76
* ``ref_identity_numerator``    -- benchmarks/chunked_attention_benchmark.py:81-93
* ``ref_sliding_window_attn``   -- benchmarks/sliding_attention_benchmark.py:32-56
* ``ref_based_layer``           -- the full BASED layer of kernels/nki_attention_sliding.py:4-5,
                                   final = linear attention + sliding-window softmax

and adds the parity oracles the GPU tests compare against:

* ``based_dense``      -- dense BASED (numerator, denominator, output) evaluated in fp32 or
                          fp64 on already dtype-rounded inputs, looped per (b, h) to bound memory.
* ``based_chunked``    -- the chunk recurrence of kernels/nki_attention_chunked.py:65-109
                          (state ``S += phi(K_c)^T V_c``, inter ``phi(Q_c) S``, causal intra part)
                          extended with the K-sum ``z`` so it can also normalise.  Used as the
                          CPU baseline for long sequences and cross-checked against
                          ``based_dense``.
* ``sliding_dense``    -- sliding-window softmax in fp32/fp64 (same math as
                          ``ref_sliding_window_attn`` without the final cast).
* ``based_loops`` / ``sliding_loops`` -- pure-Python brute force for tiny inputs.
* ``make_inputs``      -- the seeded synthetic inputs of the benchmark configurations.

Every function here is pinned by tests/test_oracle.py against brute force, closed forms,
identities and library routines; the reference ships no golden vectors of its own.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

EPS = 1e-6


# ----------------------------------------------------------------------------------------
# Restatements of the reference's PyTorch functions
# ----------------------------------------------------------------------------------------

def ref_based_attn(q, k, v, eps=EPS):
    """kernels/pytorch_attention.py:27-42.

    The 1/sqrt(d) scale is applied to q only (:33-35); the polynomial 1 + s + s^2/2 (:36),
    the ``tril(ones)`` mask (:38), the row sum + eps (:40) and the final matmul / divide (:41)
    all run in q's dtype, exactly as in the reference.
    """
    d = q.shape[-1]
    scale = 1.0 / math.sqrt(d)
    scores = torch.matmul(q * scale, k.transpose(-2, -1))
    poly = 1.0 + scores + 0.5 * scores * scores
    t = q.shape[-2]
    mask = torch.tril(torch.ones(t, t, device=q.device, dtype=q.dtype))
    masked = poly * mask
    den = masked.sum(dim=-1, keepdim=True) + eps
    return torch.matmul(masked, v) / den


def _flatten_diag_outer_product_off1(x):
    """benchmarks/chunked_attention_benchmark.py:23-31: strict upper triangle and diagonal
    of x x^T, the triangle in ``torch.triu_indices(d, d, 1)`` (row-major) order."""
    z = torch.einsum("...i,...j->...ij", x, x)
    n = z.size(-1)
    tri_i, tri_j = torch.triu_indices(n, n, 1, device=x.device)
    diag_idx = torch.arange(n, device=x.device, dtype=torch.long)
    return z[..., tri_i, tri_j], z[..., diag_idx, diag_idx]


def taylor_feature_map(x):
    """benchmarks/chunked_attention_benchmark.py:34-53.

    phi(x) = [1, x / d^(1/4), x_i^2 / (sqrt(d) sqrt(2)), x_i x_j / sqrt(d) (i<j)], so that
    phi(q) . phi(k) = 1 + s + s^2/2 with s = q.k / sqrt(d).  Dimension 1 + d + d(d+1)/2.
    """
    d = x.shape[-1]
    r2 = math.sqrt(2.0)
    rd = math.sqrt(d)
    rrd = math.sqrt(rd)
    x2_1, x2_2 = _flatten_diag_outer_product_off1(x)
    return torch.cat([torch.ones_like(x[..., 0:1]), x / rrd, x2_2 / (rd * r2), x2_1 / rd], dim=-1)


def feature_dim(d: int) -> int:
    """Length of ``taylor_feature_map`` output (benchmarks/baremetal_benchmark.py:227 uses
    1 + d + d(d+1)/2 = 2145 at d=64)."""
    return 1 + d + d * (d + 1) // 2


def ref_based_attn_phi(q, k, v, eps=EPS):
    """benchmarks/chunked_attention_benchmark.py:55-65 (named ``ref_based_attn`` there):
    dense normalised output through the feature map, fp32 inside, cast back to q.dtype."""
    q_phi = taylor_feature_map(q.float())
    k_phi = taylor_feature_map(k.float())
    scores = torch.matmul(q_phi, k_phi.transpose(-2, -1))
    t = q.shape[-2]
    mask = torch.tril(torch.ones(t, t, device=q.device, dtype=scores.dtype))
    masked = scores * mask
    den = masked.sum(dim=-1, keepdim=True) + eps
    out = torch.matmul(masked, v.float()) / den
    return out.to(q.dtype)


def ref_based_numerator(q, k, v):
    """benchmarks/chunked_attention_benchmark.py:68-76: numerator only, fp32 inside."""
    q_phi = taylor_feature_map(q.float())
    k_phi = taylor_feature_map(k.float())
    scores = torch.matmul(q_phi, k_phi.transpose(-2, -1))
    t = q.shape[-2]
    mask = torch.tril(torch.ones(t, t, device=q.device, dtype=scores.dtype))
    out = torch.matmul(scores * mask, v.float())
    return out.to(q.dtype)


def ref_identity_numerator(q, k, v):
    """benchmarks/chunked_attention_benchmark.py:81-93: causal identity-map linear
    attention numerator (no polynomial), in q's dtype."""
    d = q.shape[-1]
    scale = 1.0 / math.sqrt(d)
    scores = torch.matmul(q * scale, k.transpose(-2, -1))
    t = q.shape[-2]
    mask = torch.tril(torch.ones(t, t, device=q.device, dtype=q.dtype))
    return torch.matmul(scores * mask, v)


def ref_sliding_window_attn(q, k, v, window_size=64, eps=EPS):
    """benchmarks/sliding_attention_benchmark.py:32-56.

    q is scaled by 1/sqrt(d) in fp32 (:39-40); key u is visible to query t iff
    t - W + 1 <= u <= t (:46-51); invalid scores are -inf (:53), softmax (:54), @ v in fp32
    (:55), cast to q.dtype (:56).  ``eps`` is accepted and unused, as in the reference.
    """
    b, h, t, d = q.shape
    scale = 1.0 / math.sqrt(d)
    q_s = q.float() * scale
    scores = torch.matmul(q_s, k.float().transpose(-2, -1))
    row_idx = torch.arange(t, device=q.device).unsqueeze(1)
    col_idx = torch.arange(t, device=q.device).unsqueeze(0)
    mask = (col_idx <= row_idx) & (col_idx >= (row_idx - window_size + 1))
    scores = scores.masked_fill(~mask.unsqueeze(0).unsqueeze(0), float("-inf"))
    weights = torch.softmax(scores, dim=-1)
    out = torch.matmul(weights, v.float())
    return out.to(q.dtype)


def ref_based_layer(q, k, v, window_size=64, q_sw=None, k_sw=None, eps=EPS):
    """kernels/nki_attention_sliding.py:4-5: final = linear_attention(Q, K, V) +
    sliding_window_softmax(Q, K, V), each branch as the reference computes it
    (``ref_based_attn`` and ``ref_sliding_window_attn``, both in q's dtype), summed in that
    dtype.  ``q_sw`` / ``k_sw`` give the softmax branch its own projections (default q, k)."""
    q_sw = q if q_sw is None else q_sw
    k_sw = k if k_sw is None else k_sw
    return ref_based_attn(q, k, v, eps=eps) + ref_sliding_window_attn(q_sw, k_sw, v, window_size=window_size)


def based_layer_dense(q, k, v, window_size=64, q_sw=None, k_sw=None, eps=EPS, dtype=torch.float64):
    """The same layer in ``dtype`` on already rounded inputs: ``based_dense`` + ``sliding_dense``."""
    q_sw = q if q_sw is None else q_sw
    k_sw = k if k_sw is None else k_sw
    y, _, _ = based_dense(q, k, v, eps=eps, dtype=dtype)
    return y + sliding_dense(q_sw, k_sw, v, window_size=window_size, dtype=dtype)


# ----------------------------------------------------------------------------------------
# Parity oracles (higher precision, looped to bound memory)
# ----------------------------------------------------------------------------------------

def based_dense(q, k, v, eps=EPS, dtype=torch.float64, scale=None):
    """Dense BASED in ``dtype`` on the given (already rounded) inputs.

    Same math as kernels/pytorch_attention.py:33-41 -- s = (q*scale).k, p = 1 + s + s^2/2,
    causal mask, den = sum p + eps, y = (p @ v) / den -- but evaluated in fp32/fp64 and
    looped over (b, h) so that only one t x t temporary is live.

    Returns ``(y, num, den)`` with ``den`` *without* eps, shapes (b,h,t,dv), (b,h,t,dv),
    (b,h,t).
    """
    b, h, t, d = q.shape
    dv = v.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    num = torch.empty(b, h, t, dv, dtype=dtype)
    den = torch.empty(b, h, t, dtype=dtype)
    mask = torch.tril(torch.ones(t, t, dtype=dtype))
    for bi in range(b):
        for hi in range(h):
            qq = q[bi, hi].to(dtype) * scale
            kk = k[bi, hi].to(dtype)
            vv = v[bi, hi].to(dtype)
            s = qq @ kk.T
            p = (1.0 + s + 0.5 * s * s) * mask
            num[bi, hi] = p @ vv
            den[bi, hi] = p.sum(-1)
    y = num / (den + eps).unsqueeze(-1)
    return y, num, den


def phi_pow_scale(x, scale):
    """phi-form of the polynomial kernel for a general score scale: phi(q).phi(k) =
    1 + scale*(q.k) + (scale*(q.k))^2 / 2.  With scale = 1/sqrt(d) this equals
    ``taylor_feature_map`` (same element order)."""
    d = x.shape[-1]
    tri_i, tri_j = torch.triu_indices(d, d, 1)
    x2 = x.unsqueeze(-1) * x.unsqueeze(-2)
    return torch.cat(
        [
            torch.ones_like(x[..., 0:1]),
            x * math.sqrt(scale),
            x2.diagonal(dim1=-2, dim2=-1) * (scale / math.sqrt(2.0)),
            x2[..., tri_i, tri_j] * scale,
        ],
        dim=-1,
    )


def based_chunked(q, k, v, chunk=64, eps=EPS, dtype=torch.float32, normalize=True,
                  scale=None, return_state=False):
    """Chunk recurrence of kernels/nki_attention_chunked.py:65-109, in ``dtype`` on CPU.

    Per head, zero the state (:66-69); for each chunk c in order (:71):
      inter  o  = phi(Q_c) @ S                        (:95)
      scores A  = phi(Q_c) @ phi(K_c)^T, causal mask  (:98, :105-106)
      intra  o += A @ V_c                             (:107)
      update S += phi(K_c)^T @ V_c                    (:101-102)
    The reference kernel returns the numerator only; here the K-sum z (the state of the
    constant feature) is carried alongside so the same pass also yields den = phi(q).z +
    rowsum(A) and the normalised output.  ``return_state`` also returns the final
    (S, z) per head, shapes (b,h,F,dv) and (b,h,F).
    """
    b, h, t, d = q.shape
    dv = v.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    F = feature_dim(d)
    out = torch.empty(b, h, t, dv, dtype=dtype)
    states = torch.empty(b, h, F, dv, dtype=dtype) if return_state else None
    zs = torch.empty(b, h, F, dtype=dtype) if return_state else None
    for bi in range(b):
        for hi in range(h):
            qf = phi_pow_scale(q[bi, hi].to(dtype), scale)
            kf = phi_pow_scale(k[bi, hi].to(dtype), scale)
            vv = v[bi, hi].to(dtype)
            S = torch.zeros(F, dv, dtype=dtype)
            z = torch.zeros(F, dtype=dtype)
            for c0 in range(0, t, chunk):
                c1 = min(c0 + chunk, t)
                qc, kc, vc = qf[c0:c1], kf[c0:c1], vv[c0:c1]
                a = torch.tril(qc @ kc.T)
                o = qc @ S + a @ vc
                if normalize:
                    den = qc @ z + a.sum(-1)
                    o = o / (den + eps).unsqueeze(-1)
                out[bi, hi, c0:c1] = o
                S = S + kc.T @ vc
                z = z + kc.sum(0)
            if return_state:
                states[bi, hi] = S
                zs[bi, hi] = z
    if return_state:
        return out, states, zs
    return out


def sliding_dense(q, k, v, window_size=64, dtype=torch.float64, scale=None):
    """Sliding-window softmax attention in ``dtype`` (benchmarks/sliding_attention_benchmark.py
    :32-55 without the final cast), looped per (b, h)."""
    b, h, t, d = q.shape
    dv = v.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    row = torch.arange(t).unsqueeze(1)
    col = torch.arange(t).unsqueeze(0)
    valid = (col <= row) & (col >= row - window_size + 1)
    out = torch.empty(b, h, t, dv, dtype=dtype)
    for bi in range(b):
        for hi in range(h):
            s = (q[bi, hi].to(dtype) * scale) @ k[bi, hi].to(dtype).T
            s = s.masked_fill(~valid, float("-inf"))
            out[bi, hi] = torch.softmax(s, dim=-1) @ v[bi, hi].to(dtype)
    return out


def sliding_banded(q, k, v, window_size=64, dtype=torch.float32, scale=None, block=512):
    """Sliding-window softmax computed on row blocks with only the keys each block can see
    (keys [r0 - W + 1, r1)), so long sequences never build a t x t matrix.  Same math as
    ``sliding_dense``; used for the CPU baseline at full size."""
    b, h, t, d = q.shape
    dv = v.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    out = torch.empty(b, h, t, dv, dtype=dtype)
    qs = q.to(dtype) * scale
    kk = k.to(dtype)
    vv = v.to(dtype)
    for r0 in range(0, t, block):
        r1 = min(r0 + block, t)
        c0 = max(0, r0 - window_size + 1)
        row = torch.arange(r0, r1).unsqueeze(1)
        col = torch.arange(c0, r1).unsqueeze(0)
        valid = (col <= row) & (col >= row - window_size + 1)
        s = qs[:, :, r0:r1] @ kk[:, :, c0:r1].transpose(-2, -1)
        s = s.masked_fill(~valid, float("-inf"))
        out[:, :, r0:r1] = torch.softmax(s, dim=-1) @ vv[:, :, c0:r1]
    return out


# ----------------------------------------------------------------------------------------
# Brute force (tiny inputs only)
# ----------------------------------------------------------------------------------------

def based_loops(q, k, v, eps=EPS):
    """Pure-Python fp64 BASED, straight from the definition: for each (b,h,t),
    y_t = sum_{u<=t} p(s_tu) v_u / (sum_{u<=t} p(s_tu) + eps), p(s) = 1 + s + s^2/2,
    s_tu = (q_t . k_u)/sqrt(d)."""
    qa = np.asarray(q, dtype=np.float64)
    ka = np.asarray(k, dtype=np.float64)
    va = np.asarray(v, dtype=np.float64)
    b, h, t, d = qa.shape
    dv = va.shape[-1]
    out = np.zeros((b, h, t, dv))
    for bi in range(b):
        for hi in range(h):
            for ti in range(t):
                acc = [0.0] * dv
                z = 0.0
                for ui in range(ti + 1):
                    s = sum(qa[bi, hi, ti, e] * ka[bi, hi, ui, e] for e in range(d)) / math.sqrt(d)
                    p = 1.0 + s + 0.5 * s * s
                    z += p
                    for e in range(dv):
                        acc[e] += p * va[bi, hi, ui, e]
                for e in range(dv):
                    out[bi, hi, ti, e] = acc[e] / (z + eps)
    return out


def sliding_loops(q, k, v, window_size):
    """Pure-Python fp64 sliding-window softmax from the definition."""
    qa = np.asarray(q, dtype=np.float64)
    ka = np.asarray(k, dtype=np.float64)
    va = np.asarray(v, dtype=np.float64)
    b, h, t, d = qa.shape
    dv = va.shape[-1]
    out = np.zeros((b, h, t, dv))
    for bi in range(b):
        for hi in range(h):
            for ti in range(t):
                lo = max(0, ti - window_size + 1)
                ss = [sum(qa[bi, hi, ti, e] * ka[bi, hi, u, e] for e in range(d)) / math.sqrt(d)
                      for u in range(lo, ti + 1)]
                m = max(ss)
                w = [math.exp(s - m) for s in ss]
                tot = sum(w)
                for e in range(dv):
                    out[bi, hi, ti, e] = sum(w[j] * va[bi, hi, lo + j, e] for j in range(len(w))) / tot
    return out


# ----------------------------------------------------------------------------------------
# Seeded inputs and the parity metric
# ----------------------------------------------------------------------------------------

@dataclass(frozen=True)
class Config:
    name: str
    kind: str          # "parallel" | "chunked" | "sliding"
    B: int
    H: int
    N: int
    d: int
    dv: int
    dtype: torch.dtype
    seed: int
    chunk: int = 64
    window: int = 64
    prescale: bool = True   # q, k /= sqrt(d) before the op (BASED configs)


CONFIGS = {
    "parallel_fp32_b1h4n1024": Config("parallel_fp32_b1h4n1024", "parallel", 1, 4, 1024, 16, 64, torch.float32, 0),
    "parallel_bf16_b2h16n2048": Config("parallel_bf16_b2h16n2048", "parallel", 2, 16, 2048, 16, 64, torch.bfloat16, 1),
    "chunked_bf16_b2h16n8192": Config("chunked_bf16_b2h16n8192", "chunked", 2, 16, 8192, 16, 64, torch.bfloat16, 2, chunk=64),
    "sliding_w64_bf16_b2h16n4096": Config("sliding_w64_bf16_b2h16n4096", "sliding", 2, 16, 4096, 64, 64, torch.bfloat16, 3,
                              window=64, prescale=False),
    "chunked_bf16_b1h16n65536": Config("chunked_bf16_b1h16n65536", "chunked", 1, 16, 65536, 16, 64, torch.bfloat16, 4,
                                   chunk=128),
}


def make_inputs(B, H, N, d, dv, dtype, seed, prescale=True):
    """Seeded CPU inputs drawn in the reference's order q, k, v
    (benchmarks/chunked_attention_benchmark.py:158-160), N(0,1); for the BASED configurations
    q and k are then divided by sqrt(d) (the op applies its own 1/sqrt(d) afterwards), and
    everything is cast to ``dtype``."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, N, d, generator=g)
    k = torch.randn(B, H, N, d, generator=g)
    v = torch.randn(B, H, N, dv, generator=g)
    if prescale:
        q = q / math.sqrt(d)
        k = k / math.sqrt(d)
    return q.to(dtype), k.to(dtype), v.to(dtype)


def config_inputs(cfg: Config, prescale=None):
    return make_inputs(cfg.B, cfg.H, cfg.N, cfg.d, cfg.dv, cfg.dtype, cfg.seed,
                       cfg.prescale if prescale is None else prescale)


def rel_err(y, ref):
    """Parity metric: max |y - ref| / rms(ref), computed in fp64."""
    y = torch.as_tensor(y).double()
    ref = torch.as_tensor(ref).double()
    rms = ref.pow(2).mean().sqrt().item()
    return (y - ref).abs().max().item() / max(rms, 1e-300)


TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}
