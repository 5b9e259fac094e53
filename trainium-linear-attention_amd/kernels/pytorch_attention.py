"""Fused causal BASED attention on MI355X -- drop-in for kernels/pytorch_attention.py.

Same entry points and argument meaning as the reference module (Willy-Chan/
trainium-linear-attention, kernels/pytorch_attention.py):

* ``solution_nki(q, k, v, eps=1e-6)``  (reference :44-78)  -- the fused kernel path.
* ``solution(q, k, v, eps=1e-6)``      (reference :81-92)  -- dispatcher.

q, k: (b, h, t, d); v: (b, h, t, dv); output (b, h, t, dv) in q's dtype.  The math is
kernels/pytorch_attention.py:33-41: s = (q/sqrt(d)).k, p = 1 + s + s^2/2, causal,
y = (p @ v) / (sum p + eps).

Behavioural differences, all deliberate:
* there is no PyTorch fallback: tensors must be on a ROCm device and errors raise
  (the reference's ``solution`` swallows kernel exceptions, :87-92);
* dv may differ from d (the reference wrapper reshapes v to d, :60);
* no padding copies: ragged t, any d <= 128 and dv <= 128 are handled in-kernel.

``ref_based_attn(q, k, v, eps=1e-6)`` keeps the reference's name (:27-42) so that its callers'
``from kernels.pytorch_attention import ref_based_attn, solution_nki`` resolves; on GPU
tensors it runs the fused kernel, i.e. it is the same computation as ``solution_nki`` and not
an independent check.  The reference's dense PyTorch restatement used as the test oracle lives
outside this package.
"""

from __future__ import annotations

import math

import torch

from . import _lib

__all__ = ["solution_nki", "solution", "based_parallel", "ref_based_attn"]


def _compute_dtype(dt: torch.dtype) -> torch.dtype:
    if dt in (torch.bfloat16, torch.float32):
        return dt
    if dt in (torch.float16, torch.float64):
        return torch.float32
    raise _lib.BasedLAError(f"unsupported input dtype {dt}")


def _check_qkv(q, k, v):
    _lib.require_gpu(q, k, v)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise _lib.BasedLAError("q, k, v must be 4-D (b, h, t, d)")
    if k.shape != q.shape:
        raise _lib.BasedLAError(f"k shape {tuple(k.shape)} must equal q shape {tuple(q.shape)}")
    if v.shape[:3] != q.shape[:3]:
        raise _lib.BasedLAError(f"v shape {tuple(v.shape)} must match q in (b, h, t)")
    if not (q.dtype == k.dtype == v.dtype):
        raise _lib.BasedLAError("q, k, v must share one dtype")


def _as_kernel_input(x: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    """x in dtype dt, contiguous and 16-byte aligned (the kernels copy rows 16 bytes at a time)."""
    if x.dtype != dt:
        x = x.to(dt)
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    return x


def based_parallel(q, k, v, eps=1e-6, scale=None, normalize=True, out_dtype=None, return_den=False):
    """Parallel (quadratic) fused BASED attention through ``la_based_parallel_fwd``.

    ``scale`` defaults to 1/sqrt(d) (reference :34); ``normalize=False`` returns the
    numerator; ``out_dtype`` defaults to q.dtype (fp32 is used internally for fp16/fp64);
    ``return_den`` also returns the fp32 denominator sum_{u<=t} p_tu (without eps), as the
    NKI kernel does (kernels/nki_attention.py:107-108).
    """
    _check_qkv(q, k, v)
    b, h, t, d = q.shape
    dv = v.shape[-1]
    cdt = _compute_dtype(q.dtype)
    odt = q.dtype if out_dtype is None else out_dtype
    kdt = odt if odt in (torch.float32, torch.bfloat16) else torch.float32
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    qc, kc, vc = (_as_kernel_input(x, cdt) for x in (q, k, v))
    out = torch.empty(b, h, t, dv, dtype=kdt, device=q.device)
    den = torch.empty(b, h, t, dtype=torch.float32, device=q.device) if return_den else None
    L = _lib.lib()
    ws_bytes = int(L.la_based_parallel_workspace_bytes(b, h, t, d, dv, _lib.dtype_code(cdt)))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    rc = L.la_based_parallel_fwd(
        _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.dtype_code(cdt), _lib.ptr(out), _lib.dtype_code(kdt),
        _lib.ptr(den), b, h, t, d, dv, float(scale), float(eps), 1 if normalize else 0, _lib.ptr(ws), ws_bytes,
        _lib.stream_of(q))
    _lib.check(rc, "la_based_parallel_fwd")
    if out.dtype != odt:
        out = out.to(odt)
    return (out, den) if return_den else out


def solution_nki(q, k, v, eps=1e-6):
    """BASED causal attention via the fused MI355X kernel (reference :44-78).

    q, k: (b, h, t, d); v: (b, h, t, dv).  Returns (b, h, t, dv) in q.dtype.
    """
    return based_parallel(q, k, v, eps=eps)


def ref_based_attn(q, k, v, eps=1e-6):
    """The reference's ``ref_based_attn`` entry point (:27-42), run by the fused kernel.

    Same signature and function (s = (q/sqrt(d)).k, p = 1 + s + s^2/2, causal,
    y = (p @ v) / (sum p + eps), output in q.dtype); computed on the GPU by
    ``la_based_parallel_fwd`` with fp32 accumulation instead of the reference's
    input-dtype arithmetic.  Tensors must be on a ROCm device.
    """
    return based_parallel(q, k, v, eps=eps)


# Sequence length from which ``solution`` uses the chunked (linear-time) kernel.  Measured on
# MI355X at d=16, dv=64, bf16 (B1 H2, B2 H16, B8 H16; N = 256 .. 16384, whole forward of each
# path): the chunked forward was faster at every length, from 0.014 vs 0.015 ms at N=256 to
# 0.084 vs 0.762 ms at B2 H16 N=16384; shorter sequences were not measured and stay on the
# fused kernel.
CHUNKED_MIN_T = 256

# Sequence length from which ``solution`` uses the segment-state chunked path for the other head
# dims and for fp32 inputs (d <= 64, dv <= 128).  Measured on MI355X at N = 8192, B2 H16 (whole
# calls, ms, chunked / fused): bf16 d64 dv64 0.435 / 0.451, bf16 d32 dv128 0.517 / 0.511, fp32
# d16 dv64 0.774 / 1.455; the fused kernel's work grows with N^2, the chunked paths' with N.
GENERAL_CHUNKED_MIN_T = 16384


def solution(q, k, v, eps=1e-6):
    """BASED causal attention (reference :81-92).

    Dispatches by sequence length between the parallel fused kernel and the chunked kernels,
    which compute the same function: the d = 16 recurrence kernel from ``CHUNKED_MIN_T`` tokens,
    the segment-state path for other head dims and fp32 inputs from ``GENERAL_CHUNKED_MIN_T``;
    shorter sequences and other shapes go to the fused kernel.  There is no PyTorch fallback.
    """
    from .chunked_attention import chunked_based_attn, chunked_supported, general_chunked_supported
    t, d, dv = q.shape[-2], q.shape[-1], v.shape[-1]
    cdt = _compute_dtype(q.dtype)
    if (t >= CHUNKED_MIN_T and chunked_supported(d, dv, cdt)) or (
            t >= GENERAL_CHUNKED_MIN_T and general_chunked_supported(d, dv, cdt)):
        return chunked_based_attn(q, k, v, eps=eps)
    return based_parallel(q, k, v, eps=eps)
