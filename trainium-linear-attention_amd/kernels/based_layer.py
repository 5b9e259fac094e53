"""The full BASED layer on MI355X: causal linear attention plus sliding-window softmax attention,
final = linear_attention(Q, K, V) + sliding_window_softmax(Q, K, V)
(kernels/nki_attention_sliding.py:4-5, where the reference describes the sliding kernel as the
third component of full BASED attention; it computes the two branches in separate calls).

The two branches may use different head dims: the linear branch takes the feature projections
q, k (d = 16 in BASED), the softmax branch its own q_sw, k_sw (any d_sw <= 128; default q, k),
and both attend over the same v.  The linear branch runs first, into fp32, on the kernel
``solution`` would pick (chunked from ``CHUNKED_MIN_T`` tokens when bf16, d = 16, dv <= 64,
else the fused parallel kernel); the sliding-window kernel then adds that fp32 result in its
store (``la_sliding_window_fwd_add``) and rounds the sum once to the output dtype, so the sum
costs no separate pass over the output.
"""

from __future__ import annotations

import torch

from . import _lib, pytorch_attention
from .chunked_attention import based_chunked, chunked_supported
from .pytorch_attention import _check_qkv, _compute_dtype, based_parallel
from .sliding_attention import _sliding

__all__ = ["based_layer_attn"]


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
    if t >= pytorch_attention.CHUNKED_MIN_T and chunked_supported(d, dv, _compute_dtype(q.dtype)):
        lin = based_chunked(q, k, v, eps=eps, normalize=True, out_dtype=torch.float32)
    else:
        lin = based_parallel(q, k, v, eps=eps, out_dtype=torch.float32)
    return _sliding(q_sw, k_sw, v, window_size, None, q.dtype, lin, addend_is_scratch=True)
