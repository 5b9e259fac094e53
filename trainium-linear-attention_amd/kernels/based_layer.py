"""The full BASED layer on MI355X: causal linear attention plus sliding-window softmax attention,
final = linear_attention(Q, K, V) + sliding_window_softmax(Q, K, V)
(kernels/nki_attention_sliding.py:4-5, where the reference describes the sliding kernel as the
third component of full BASED attention; it computes the two branches in separate calls).

The two branches may use different head dims: the linear branch takes the feature projections
q, k (d = 16 in BASED), the softmax branch its own q_sw, k_sw (any d_sw <= 128; default q, k),
and both attend over the same v.

From ``CHUNKED_MIN_T`` tokens, for bf16 with d = 16, dv % 8 == 0, dv <= 64, d_sw in {16, 32, 64}
and window <= 64 (the benchmark layer), the whole layer is ``la_based_layer_fwd``: after the
chunked kernel's two state passes, one kernel computes both branches per (head, segment) and
stores their sum, rounded once.  Other layers run the linear branch into fp32 on the kernel
``solution`` would pick (the chunked kernel from ``CHUNKED_MIN_T`` tokens, else the fused parallel
kernel), then the sliding-window kernel adds that result in its store
(``la_sliding_window_fwd_add``), rounding the sum once.
"""

from __future__ import annotations

import torch

from . import _lib, pytorch_attention
from .chunked_attention import based_chunked, chunked_supported
from .pytorch_attention import _check_qkv, _compute_dtype, based_parallel
from .sliding_attention import _sliding

__all__ = ["based_layer_attn", "layer_fused_supported"]


def layer_fused_supported(d: int, dv: int, d_sw: int, window_size: int, dtype: torch.dtype) -> bool:
    """Shapes of the one-launch layer kernel (``la_based_layer_fwd``)."""
    return (dtype == torch.bfloat16 and d == 16 and dv % 8 == 0 and dv <= 64 and d_sw in (16, 32, 64)
            and 1 <= int(window_size) <= 64)


def _aligned(x: torch.Tensor) -> torch.Tensor:
    x = x.contiguous()
    return x if x.data_ptr() % 16 == 0 else x.clone()


def _layer_fused(q, k, v, q_sw, k_sw, window, eps):
    b, h, t, d = q.shape
    dv, d_sw = v.shape[-1], q_sw.shape[-1]
    qc, kc, vc, qs, ks = (_aligned(x) for x in (q, k, v, q_sw, k_sw))
    out = torch.empty(b, h, t, dv, dtype=q.dtype, device=q.device)
    L = _lib.lib()
    ws_bytes = int(L.la_based_chunked_workspace_bytes_dt(b, h, t, d, dv, 64, _lib.LA_BF16))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
    rc = L.la_based_layer_fwd(_lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.ptr(qs), _lib.ptr(ks),
                              _lib.dtype_code(q.dtype), _lib.ptr(out), _lib.dtype_code(out.dtype), b, h, t, d, dv,
                              d_sw, window, 1.0 / d ** 0.5, 1.0 / d_sw ** 0.5, float(eps), _lib.ptr(ws), ws_bytes,
                              _lib.stream_of(q))
    _lib.check(rc, "la_based_layer_fwd")
    return out


def based_layer_attn(q, k, v, window_size=64, q_sw=None, k_sw=None, eps=1e-6):
    """linear_attention(q, k, v) + sliding_window_softmax(q_sw, k_sw, v); returns q.dtype.

    q, k: (b, h, t, d); v: (b, h, t, dv); q_sw, k_sw: (b, h, t, d_sw), default q and k.
    Scales: 1/sqrt(d) in the linear branch, 1/sqrt(d_sw) in the softmax branch.
    """
    q_sw = q if q_sw is None else q_sw
    k_sw = k if k_sw is None else k_sw
    _check_qkv(q, k, v)
    _check_qkv(q_sw, k_sw, v)
    if q_sw.dtype != q.dtype:
        raise _lib.BasedLAError("q_sw, k_sw must have q's dtype")
    if int(window_size) < 1:
        raise _lib.BasedLAError("window_size must be >= 1")
    t, d, dv = q.shape[-2], q.shape[-1], v.shape[-1]
    if t >= pytorch_attention.CHUNKED_MIN_T and layer_fused_supported(d, dv, q_sw.shape[-1], window_size, q.dtype):
        return _layer_fused(q, k, v, q_sw, k_sw, int(window_size), eps)
    if t >= pytorch_attention.CHUNKED_MIN_T and chunked_supported(d, dv, _compute_dtype(q.dtype)):
        lin = based_chunked(q, k, v, eps=eps, normalize=True, out_dtype=torch.float32)
    else:
        lin = based_parallel(q, k, v, eps=eps, out_dtype=torch.float32)
    return _sliding(q_sw, k_sw, v, window_size, None, q.dtype, lin, addend_is_scratch=True)
