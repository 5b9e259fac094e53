"""Chunked recurrent BASED attention and the Taylor feature map on MI355X -- drop-in for the
reference's ``taylor_feature_map`` and ``chunked_nki_numerator``
(benchmarks/chunked_attention_benchmark.py:34-53, :96-126).

* ``taylor_feature_map(x)`` -- phi(x) = [1, x/d^(1/4), x_i^2/(sqrt(d) sqrt(2)), x_i x_j/sqrt(d)]
  (i < j in triu order), computed by a HIP kernel; returns x.dtype.
* ``chunked_nki_numerator(q, k, v, chunk_size=64)`` -- numerator only, as the NKI kernel
  returns (kernels/nki_attention_chunked.py:56).
* ``chunked_based_attn(q, k, v, chunk_size=64, eps=1e-6)`` -- the same recurrence carrying the
  K-sum so it also normalises; equal to ``solution_nki`` up to rounding.

The feature map is applied inside the chunked kernel: phi(Q), phi(K) never reach HBM, and the
state stays on chip across chunks (the NKI kernel round-trips it through HBM,
kernels/nki_attention_chunked.py:92-102).  dv may differ from d.

Two chunked paths: the recurrence kernel for bf16 inputs with d = 16 and dv <= 64 (the BASED
configuration), and for other head dims and fp32 inputs (d <= 64, dv <= 128) a segment-state
path (state prefixes of 512-token segments in the feature basis, then every query's contraction
with its segment's prefix plus the quadratic form inside the segment; fp32 throughout for fp32
inputs).  Both are linear in the sequence
length.  Shapes outside both are computed by the fused parallel kernel, which evaluates the same
function (numerator or normalised) on the GPU.  ``chunk_size`` is the reference's argument
(any value >= 1); the kernel's recurrence runs 128-token chunks (``la_based_chunked_chunk_used``
reports it), which gives the same result for every chunk size up to rounding (chunk-size
invariance of the recurrence).
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .pytorch_attention import _as_kernel_input, _check_qkv, _compute_dtype

__all__ = ["taylor_feature_map", "feature_dim", "chunked_nki_numerator", "chunked_based_attn", "based_chunked",
           "based_decode_step", "chunked_supported", "general_chunked_supported"]


def feature_dim(d: int) -> int:
    return 1 + d + d * (d + 1) // 2


def taylor_feature_map(x):
    """phi(x) for x of shape (..., d); output (..., 1 + d + d(d+1)/2) in x.dtype."""
    _lib.require_gpu(x)
    d = x.shape[-1]
    cdt = _compute_dtype(x.dtype)
    kdt = x.dtype if x.dtype in (torch.float32, torch.bfloat16) else torch.float32
    xc = _as_kernel_input(x, cdt)
    rows = xc.numel() // d if d > 0 else 0
    out = torch.empty(*x.shape[:-1], feature_dim(d), dtype=kdt, device=x.device)
    rc = _lib.lib().la_taylor_feature_map(_lib.ptr(xc), _lib.dtype_code(cdt), _lib.ptr(out), _lib.dtype_code(kdt),
                                          rows, d, _lib.stream_of(x))
    _lib.check(rc, "la_taylor_feature_map")
    return out if out.dtype == x.dtype else out.to(x.dtype)


def chunked_supported(d: int, dv: int, dtype: torch.dtype) -> bool:
    """Shapes the chunk-recurrence kernel implements (bf16, d = 16, dv <= 64); it also exports
    and imports states."""
    return d == 16 and 1 <= dv <= 64 and dtype == torch.bfloat16


def general_chunked_supported(d: int, dv: int, dtype: torch.dtype) -> bool:
    """Shapes of the segment-state chunked path (bf16 or fp32, d <= 64, dv <= 128), linear in N."""
    return 1 <= d <= 64 and 1 <= dv <= 128 and dtype in (torch.bfloat16, torch.float32)


def based_chunked(q, k, v, chunk_size=64, eps=1e-6, scale=None, normalize=True, out_dtype=None,
                  return_state=False, state_in=None, prev_tokens=None):
    """Chunked recurrent BASED attention through ``la_based_chunked_fwd``.

    ``return_state`` also returns the final per-head state in the reference feature basis:
    (b, h, F, dv + 1) fp32 = [sum_u phi(k_u) v_u^T | sum_u phi(k_u)].
    ``state_in`` (same layout, e.g. an earlier call's state) continues a sequence: these tokens
    follow the ``prev_tokens`` tokens it summarises (default: its count entry z[0] of head 0,
    read back to the host), through ``la_based_chunked_fwd_continue``; it is not modified.
    On the segment-state shapes (d != 16, dv > 64, fp32 inputs) both go through
    ``la_based_chunked_fwd_num_den`` and fp32 GEMMs on phi (see _segment_state_with_state),
    and the count of ``state_in`` is its own z[0] (``prev_tokens`` is not used).
    """
    _check_qkv(q, k, v)
    if int(chunk_size) < 1:
        raise _lib.BasedLAError("chunk_size must be >= 1")
    b, h, t, d = q.shape
    dv = v.shape[-1]
    cdt = _compute_dtype(q.dtype)
    with_state = return_state or state_in is not None
    if not chunked_supported(d, dv, cdt) and not general_chunked_supported(d, dv, cdt):
        if with_state:
            raise _lib.BasedLAError(f"state export and import need d <= 64, dv <= 128 (got d={d}, dv={dv})")
        from .pytorch_attention import based_parallel
        return based_parallel(q, k, v, eps=eps, scale=scale, normalize=normalize, out_dtype=out_dtype)
    odt = q.dtype if out_dtype is None else out_dtype
    kdt = odt if odt in (torch.float32, torch.bfloat16) else torch.float32
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    qc, kc, vc = (_as_kernel_input(x, cdt) for x in (q, k, v))
    if with_state and not chunked_supported(d, dv, cdt):
        out, state = _segment_state_with_state(qc, kc, vc, cdt, kdt, int(chunk_size), float(scale), float(eps),
                                               normalize, return_state, state_in)
        if out.dtype != odt:
            out = out.to(odt)
        return (out, state) if return_state else out
    out = torch.empty(b, h, t, dv, dtype=kdt, device=q.device)
    L = _lib.lib()
    ws_bytes = int(L.la_based_chunked_workspace_bytes_dt(b, h, t, d, dv, int(chunk_size), _lib.dtype_code(cdt)))
    if ws_bytes == (1 << 64) - 1:
        raise _lib.BasedLAError(f"chunked kernel does not support d={d}, dv={dv}, chunk={chunk_size}")
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    state = torch.empty(b, h, feature_dim(d), dv + 1, dtype=torch.float32, device=q.device) if return_state else None
    if state_in is None:
        rc = L.la_based_chunked_fwd(
            _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.dtype_code(cdt), _lib.ptr(out), _lib.dtype_code(kdt),
            b, h, t, d, dv, int(chunk_size), float(scale), float(eps), 1 if normalize else 0,
            _lib.ptr(ws), ws_bytes, _lib.ptr(state), _lib.stream_of(q))
        _lib.check(rc, "la_based_chunked_fwd")
    else:
        _lib.require_gpu(q, state_in)
        if state_in.dtype != torch.float32 or tuple(state_in.shape) != (b, h, feature_dim(d), dv + 1):
            raise _lib.BasedLAError(f"state_in must be fp32 {(b, h, feature_dim(d), dv + 1)}")
        si = state_in.contiguous()
        if prev_tokens is None:
            prev_tokens = int(round(float(si[0, 0, 0, dv].item()))) if b * h > 0 else 0
        rc = L.la_based_chunked_fwd_continue(
            _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.dtype_code(cdt), _lib.ptr(out), _lib.dtype_code(kdt),
            b, h, t, d, dv, int(chunk_size), float(scale), float(eps), 1 if normalize else 0,
            _lib.ptr(ws), ws_bytes, _lib.ptr(si), int(prev_tokens), _lib.ptr(state), _lib.stream_of(q))
        _lib.check(rc, "la_based_chunked_fwd_continue")
    if out.dtype != odt:
        out = out.to(odt)
    return (out, state) if return_state else out


def _phi_f32(x, a, L):
    """phi(a x) in fp32 for rows x (n, t, d) by la_taylor_feature_map; a = 1 keeps x as it is."""
    n, t, d = x.shape
    xs = x if a == 1.0 else (x.float() * a)
    out = torch.empty(n, t, feature_dim(d), dtype=torch.float32, device=x.device)
    if n * t == 0:
        return out
    rc = L.la_taylor_feature_map(_lib.ptr(xs), _lib.dtype_code(xs.dtype), _lib.ptr(out), _lib.LA_F32, n * t, d,
                                 _lib.stream_of(x))
    _lib.check(rc, "la_taylor_feature_map")
    return out


# fp32 phi(Q) / phi(K) of at most this many bytes per pass over a group of heads
_PHI_BYTES = 1 << 30


def _segment_state_with_state(qc, kc, vc, cdt, kdt, chunk, scale, eps, normalize, return_state, state_in):
    """State export and import for the segment-state shapes (d != 16, dv > 64 or fp32 inputs).

    The kernels of la_based_chunked_fwd_num_den give every row's numerator and denominator over
    these tokens from a zero state; the state enters as plain fp32 GEMMs in the reference
    feature basis, with phi from la_taylor_feature_map at phi(a x), a = (scale^2 d)^(1/4), so
    that phi(a q) . phi(a k) = 1 + s + s^2 / 2 for s = scale q.k (a = 1 at scale = 1/sqrt(d)):
      import:  num += phi(a Q) S_in[:, :dv],  den += phi(a Q) S_in[:, dv]   (every query row)
      export:  [S | z] = S_in + phi(a K)^T [V | 1]
    The layout of the states is the recurrence path's ((b, h, F, dv + 1), fp32), so states pass
    between the two paths and to based_decode_step (which evaluates phi at scale 1/sqrt(d)).  The
    token count of state_in is its own z[0]; no separate count is needed.
    """
    b, h, t, d = qc.shape
    dv = vc.shape[-1]
    F = feature_dim(d)
    dev = qc.device
    L = _lib.lib()
    rows = b * h
    a = math.sqrt(scale * math.sqrt(d))
    if abs(a - 1.0) < 1e-7:
        a = 1.0
    if state_in is not None:
        _lib.require_gpu(qc, state_in)
        if state_in.dtype != torch.float32 or tuple(state_in.shape) != (b, h, F, dv + 1):
            raise _lib.BasedLAError(f"state_in must be fp32 {(b, h, F, dv + 1)}")
        sin = state_in.contiguous().view(rows, F, dv + 1)
    ws_bytes = int(L.la_based_chunked_workspace_bytes_dt(b, h, t, d, dv, chunk, _lib.dtype_code(cdt)))
    if ws_bytes == (1 << 64) - 1:
        raise _lib.BasedLAError(f"chunked kernel does not support d={d}, dv={dv}, chunk={chunk}")
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    if state_in is None:
        out = torch.empty(b, h, t, dv, dtype=kdt, device=dev)
        rc = L.la_based_chunked_fwd(
            _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.dtype_code(cdt), _lib.ptr(out), _lib.dtype_code(kdt),
            b, h, t, d, dv, chunk, scale, eps, 1 if normalize else 0, _lib.ptr(ws), ws_bytes, None,
            _lib.stream_of(qc))
        _lib.check(rc, "la_based_chunked_fwd")
    else:
        num = torch.empty(b, h, t, dv, dtype=torch.float32, device=dev)
        den = torch.empty(b, h, t, dtype=torch.float32, device=dev)
        rc = L.la_based_chunked_fwd_num_den(
            _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.dtype_code(cdt), _lib.ptr(num), _lib.ptr(den),
            b, h, t, d, dv, chunk, scale, _lib.ptr(ws), ws_bytes, _lib.stream_of(qc))
        _lib.check(rc, "la_based_chunked_fwd_num_den")
    state = torch.empty(b, h, F, dv + 1, dtype=torch.float32, device=dev) if return_state else None
    per_head = max(1, t * F * 4)
    group = max(1, min(rows, _PHI_BYTES // per_head))
    qf, kf, vf = qc.view(rows, t, d), kc.view(rows, t, d), vc.view(rows, t, dv)
    for r0 in range(0, rows, group):
        r1 = min(rows, r0 + group)
        if state_in is not None and t > 0:
            ext = torch.bmm(_phi_f32(qf[r0:r1], a, L), sin[r0:r1])          # (n, t, dv + 1)
            num.view(rows, t, dv)[r0:r1] += ext[..., :dv]
            den.view(rows, t)[r0:r1] += ext[..., dv]
            del ext
        if return_state:
            so = state.view(rows, F, dv + 1)[r0:r1]
            if t > 0:
                vx = torch.ones(r1 - r0, dv + 1, t, dtype=torch.float32, device=dev)
                vx[:, :dv] = vf[r0:r1].transpose(1, 2)
                so.copy_(torch.bmm(vx, _phi_f32(kf[r0:r1], a, L)).transpose(1, 2))   # [V | 1]^T phi(K)
                if state_in is not None:
                    so += sin[r0:r1]
            elif state_in is not None:
                so.copy_(sin[r0:r1])
            else:
                so.zero_()
    if state_in is not None:
        out = num / (den + eps).unsqueeze(-1) if normalize else num
        if out.dtype != kdt:
            out = out.to(kdt)
    return out, state


def based_decode_step(q, k, v, state, eps=1e-6, normalize=True):
    """One decode step on an exported state (``based_chunked(..., return_state=True)``) through
    ``la_based_decode_step_ws`` (small batches split every head's state rows over several
    work-groups, with a workspace allocated here): ``state`` (b, h, F, dv + 1) fp32 = [S | z]
    is updated in place with the new token, ``[S | z] += phi(k) [v | 1]``, and the token's
    output is returned,
    ``phi(q) S / (phi(q) z + eps)`` (the numerator with ``normalize=False``), in q.dtype.

    q, k: (b, h, d) or (b, h, 1, d); v: (b, h, dv) or (b, h, 1, dv) -- one token per head.
    The reference has no decode path; this continues the chunk recurrence of
    kernels/nki_attention_chunked.py:65-109 one token at a time.
    """
    squeeze = q.dim() == 4
    if squeeze:
        if q.shape[2] != 1 or k.shape[2] != 1 or v.shape[2] != 1:
            raise _lib.BasedLAError("decode takes one token per head: shape (b, h, 1, d)")
        q, k, v = q[:, :, 0], k[:, :, 0], v[:, :, 0]
    _lib.require_gpu(q, k, v, state)
    if q.dim() != 3 or k.shape != q.shape or v.shape[:2] != q.shape[:2]:
        raise _lib.BasedLAError("q, k must be (b, h, d) and v (b, h, dv)")
    if not (q.dtype == k.dtype == v.dtype):
        raise _lib.BasedLAError("q, k, v must share one dtype")
    b, h, d = q.shape
    dv = v.shape[-1]
    if state.dtype != torch.float32 or tuple(state.shape) != (b, h, feature_dim(d), dv + 1) \
            or not state.is_contiguous():
        raise _lib.BasedLAError(f"state must be contiguous fp32 {(b, h, feature_dim(d), dv + 1)}")
    cdt = _compute_dtype(q.dtype)
    kdt = q.dtype if q.dtype in (torch.float32, torch.bfloat16) else torch.float32
    qc, kc, vc = (_as_kernel_input(x, cdt) for x in (q, k, v))
    out = torch.empty(b, h, dv, dtype=kdt, device=q.device)
    L = _lib.lib()
    ws_bytes = int(L.la_based_decode_workspace_bytes(b, h, d, dv))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes > 0 else None
    rc = L.la_based_decode_step_ws(
        _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.dtype_code(cdt), _lib.ptr(state), _lib.ptr(out),
        _lib.dtype_code(kdt), b, h, d, dv, float(eps), 1 if normalize else 0, _lib.ptr(ws), ws_bytes,
        _lib.stream_of(q))
    _lib.check(rc, "la_based_decode_step_ws")
    if out.dtype != q.dtype:
        out = out.to(q.dtype)
    return out.unsqueeze(2) if squeeze else out


def chunked_nki_numerator(q, k, v, chunk_size=64):
    """Numerator-only chunked BASED attention (reference signature); returns q.dtype."""
    return based_chunked(q, k, v, chunk_size=chunk_size, normalize=False)


def chunked_based_attn(q, k, v, chunk_size=64, eps=1e-6):
    """Normalised chunked BASED attention; returns q.dtype."""
    return based_chunked(q, k, v, chunk_size=chunk_size, eps=eps, normalize=True)
