"""Causal linear attention with the identity feature map (numerator only) on MI355X -- the
reference's ``ref_identity_numerator`` (benchmarks/chunked_attention_benchmark.py:81-93) and its
chunked NKI kernel (old/identity_linear_attn_nki_CHUNKED.py), through ``la_identity_linear_fwd``:

    y_t = sum_{u <= t} ((q_t / sqrt(d)) . k_u) v_u

The kernel takes bf16 with d in {16, 32, 64} and dv in {32, 64}; this wrapper zero-pads q and k
to the next of those d (q . k is unchanged) and runs v in column slices of at most 64, each
zero-padded to 32 or 64 (padded columns are dropped), so any d <= 64 and any dv work.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import _lib
from .pytorch_attention import _as_kernel_input, _check_qkv

__all__ = ["identity_linear_attn"]

_KERNEL_D = (16, 32, 64)


def _pad_last(x, n):
    return x if x.shape[-1] == n else F.pad(x, (0, n - x.shape[-1]))


def identity_linear_attn(q, k, v, scale=None, out_dtype=None):
    """Causal identity-map linear attention numerator; q, k (b, h, t, d), v (b, h, t, dv), bf16.

    ``scale`` defaults to 1/sqrt(d) (reference :83); returns ``out_dtype`` (default q.dtype).
    """
    _check_qkv(q, k, v)
    if q.dtype != torch.bfloat16:
        raise _lib.BasedLAError(f"the identity kernel takes bf16 inputs, got {q.dtype}")
    b, h, t, d = q.shape
    dv = v.shape[-1]
    if d > _KERNEL_D[-1]:
        raise _lib.BasedLAError(f"the identity kernel takes d <= {_KERNEL_D[-1]}, got {d}")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    odt = q.dtype if out_dtype is None else out_dtype
    kdt = odt if odt in (torch.float32, torch.bfloat16) else torch.float32
    dk = next(x for x in _KERNEL_D if x >= d)
    qc, kc = (_as_kernel_input(_pad_last(x, dk), torch.bfloat16) for x in (q, k))
    L = _lib.lib()
    out = torch.empty(b, h, t, dv, dtype=kdt, device=q.device)
    for c0 in range(0, dv, 64):
        c1 = min(dv, c0 + 64)
        w = 32 if c1 - c0 <= 32 else 64
        vc = _as_kernel_input(_pad_last(v[..., c0:c1], w), torch.bfloat16)
        oc = out if (c0, c1, w) == (0, dv, dv) else torch.empty(b, h, t, w, dtype=kdt, device=q.device)
        ws_bytes = int(L.la_identity_workspace_bytes(b, h, t, dk, w))
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
        rc = L.la_identity_linear_fwd(_lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.dtype_code(torch.bfloat16),
                                      _lib.ptr(oc), _lib.dtype_code(kdt), b, h, t, dk, w, float(scale),
                                      _lib.ptr(ws), ws_bytes, _lib.stream_of(q))
        _lib.check(rc, "la_identity_linear_fwd")
        if oc is not out:
            out[..., c0:c1] = oc[..., : c1 - c0]
    return out if out.dtype == odt else out.to(odt)
