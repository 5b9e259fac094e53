"""BASED attention layer around the MI355X kernels: the reference's module-level callers
``TrainiumBasedLinearAttention`` / ``TrainiumBasedLinearAttentionNKI``
(benchmarks/based_attention_benchmark.py:24-69) with the same constructor arguments, parameter
names (``q_proj``, ``k_proj``, ``v_proj``, ``o_proj``, bias-free ``nn.Linear(dim, dim)``) and
forward, so their state dicts load unchanged.

Steps of a forward (hidden (b, t, dim) -> (b, t, dim)):
  * one GEMM for q, k and v over the three weights concatenated (rocBLAS / hipBLASLt through
    torch); the concatenation is cached and rebuilt when a weight is replaced or changed in place;
  * its (b, t, 3, heads, head_dim) output permuted to (3, b, heads, t, head_dim) by one copy,
    so that q, k and v are contiguous per-head operands (the kernels read each head's rows
    contiguously; the wrappers then pass them on without copying);
  * the attention kernel: the fused parallel kernel (``solution_nki``, as the reference's NKI
    module) or ``solution`` (the chunked kernel from ``CHUNKED_MIN_T`` tokens);
  * the heads merged back to (b, t, dim), cast to the input dtype, and ``o_proj``.

The attention kernels are forward-only, as the reference's NKI kernel is: a backward pass that
reaches them raises instead of returning wrong gradients.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .pytorch_attention import solution, solution_nki


class _ForwardOnly(torch.autograd.Function):
    """Runs an attention kernel under autograd; its backward raises."""

    @staticmethod
    def forward(ctx, attn, q, k, v):
        return attn(q, k, v)

    @staticmethod
    def backward(ctx, grad):
        raise RuntimeError("the BASED attention kernels are forward-only: no gradient flows through them")


class TrainiumBasedLinearAttentionNKI(nn.Module):
    """BASED attention layer on the fused parallel kernel (reference :48-69).

    ``dispatch="fused"`` (default) always runs the fused parallel kernel, like the reference's NKI
    module; ``dispatch="auto"`` runs ``solution``, which takes the chunked kernel for long
    sequences.  Both compute the same function.
    """

    _DISPATCH = {"fused": solution_nki, "auto": solution}

    def __init__(self, dim: int, heads: int = 8, eps: float = 1e-6, dispatch: str = "fused"):
        super().__init__()
        self.num_heads = heads
        self.head_dim = dim // heads
        self.eps = eps
        assert dim % heads == 0
        if dispatch not in self._DISPATCH:
            raise ValueError(f"dispatch must be one of {sorted(self._DISPATCH)}, got {dispatch!r}")
        self.dispatch = dispatch
        self.q_proj = nn.Linear(dim, dim, bias=False)
        self.k_proj = nn.Linear(dim, dim, bias=False)
        self.v_proj = nn.Linear(dim, dim, bias=False)
        self.o_proj = nn.Linear(dim, dim, bias=False)
        self._wqkv = None
        self._wqkv_key = None

    def _qkv_weight(self) -> torch.Tensor:
        ws = (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight)
        if torch.is_grad_enabled() and any(w.requires_grad for w in ws):
            return torch.cat(ws, 0)     # part of the autograd graph: not cached
        key = tuple((w.data_ptr(), w._version, w.dtype, w.device) for w in ws)
        if key != self._wqkv_key:
            with torch.no_grad():
                self._wqkv = torch.cat(ws, 0)
            self._wqkv_key = key
        return self._wqkv

    def _apply(self, fn, *args, **kwargs):
        self._wqkv, self._wqkv_key = None, None   # .to() / .cuda() / .half(): rebuild the cache
        return super()._apply(fn, *args, **kwargs)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        b, t, _ = hidden_states.size()
        qkv = F.linear(hidden_states, self._qkv_weight()).view(b, t, 3, self.num_heads, self.head_dim)
        # one permuting copy to (3, b, heads, t, head_dim): q, k and v are then contiguous
        # slices, which the kernel wrappers take as they are (no copy per operand)
        q, k, v = qkv.permute(2, 0, 3, 1, 4).contiguous().unbind(0)
        kernel = self._DISPATCH[self.dispatch]
        eps = self.eps
        y = _ForwardOnly.apply(lambda q_, k_, v_: kernel(q_, k_, v_, eps=eps), q, k, v)
        y = y.transpose(1, 2).reshape(b, t, -1)
        return self.o_proj(y.to(hidden_states.dtype))


class TrainiumBasedLinearAttention(TrainiumBasedLinearAttentionNKI):
    """BASED attention layer (reference :24-45, whose forward runs the dense PyTorch
    ``ref_based_attn``): the same function on the HIP kernels, through ``solution``."""

    def __init__(self, dim: int, heads: int = 8, eps: float = 1e-6):
        super().__init__(dim, heads=heads, eps=eps, dispatch="auto")
