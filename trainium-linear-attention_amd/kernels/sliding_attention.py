"""Causal sliding-window softmax attention on MI355X -- drop-in for the reference's
``nki_sliding_window_attn`` (benchmarks/sliding_attention_benchmark.py:59-99).

Each query t attends to keys t-W+1 .. t with softmax((q/sqrt(d)).k) (reference :32-56).
Any window W >= 1 (the NKI kernel asserts W <= 65 at block 64,
kernels/nki_attention_sliding.py:50-58); dv may differ from d; no padded copies and no
mask tensor.  ``block_size`` is accepted for signature compatibility: tiling is chosen by
the kernel.  The reference's ``ref_sliding_window_attn`` is a test oracle kept outside this
package.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .pytorch_attention import _as_kernel_input, _check_qkv, _compute_dtype

__all__ = ["nki_sliding_window_attn", "sliding_window_attn"]


def sliding_window_attn(q, k, v, window_size=64, scale=None, out_dtype=None, addend=None):
    """Sliding-window softmax attention through ``la_sliding_window_fwd``.

    ``addend``: optional tensor of the output's shape, added in fp32 before the output is rounded
    (``la_sliding_window_fwd_add``); it is not modified.
    """
    return _sliding(q, k, v, window_size, scale, out_dtype, addend, addend_is_scratch=False)


def _sliding(q, k, v, window_size, scale, out_dtype, addend, addend_is_scratch):
    """``addend_is_scratch``: the caller owns an fp32 contiguous ``addend``, which then becomes the
    output buffer when the output is fp32 (the kernel reads each element before writing it)."""
    _check_qkv(q, k, v)
    if int(window_size) < 1:
        raise _lib.BasedLAError("window_size must be >= 1")
    b, h, t, d = q.shape
    dv = v.shape[-1]
    cdt = _compute_dtype(q.dtype)
    odt = q.dtype if out_dtype is None else out_dtype
    kdt = odt if odt in (torch.float32, torch.bfloat16) else torch.float32
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    qc, kc, vc = (_as_kernel_input(x, cdt) for x in (q, k, v))
    if addend is None:
        out = torch.empty(b, h, t, dv, dtype=kdt, device=q.device)
        rc = _lib.lib().la_sliding_window_fwd(
            _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.dtype_code(cdt), _lib.ptr(out), _lib.dtype_code(kdt),
            b, h, t, d, dv, int(window_size), float(scale), _lib.stream_of(q))
        _lib.check(rc, "la_sliding_window_fwd")
    else:
        _lib.require_gpu(q, addend)
        if tuple(addend.shape) != (b, h, t, dv):
            raise _lib.BasedLAError(f"addend shape {tuple(addend.shape)} must be {(b, h, t, dv)}")
        ad = _as_kernel_input(addend, torch.float32)    # addend itself when fp32, contiguous, aligned
        in_place = addend_is_scratch and ad is addend and kdt == torch.float32
        out = ad if in_place else torch.empty(b, h, t, dv, dtype=kdt, device=q.device)
        rc = _lib.lib().la_sliding_window_fwd_add(
            _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.dtype_code(cdt), _lib.ptr(ad), _lib.ptr(out),
            _lib.dtype_code(kdt), b, h, t, d, dv, int(window_size), float(scale), _lib.stream_of(q))
        _lib.check(rc, "la_sliding_window_fwd_add")
    return out if out.dtype == odt else out.to(odt)


def nki_sliding_window_attn(q, k, v, window_size=64, block_size=64):
    """Sliding-window softmax attention (reference signature); returns q.dtype."""
    if int(block_size) < 1:
        raise _lib.BasedLAError("block_size must be >= 1")
    return sliding_window_attn(q, k, v, window_size=window_size)
