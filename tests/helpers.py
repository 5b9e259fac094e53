"""Shared helpers for the GPU parity tests (inputs, oracle calls, the parity metric)."""

import os

import numpy as np
import torch

from oracle import reference as ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_golden(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as f:
        return {key: f[key] for key in f.files}


def to_dev(*xs, dtype=None):
    return tuple((x if dtype is None else x.to(dtype)).cuda() for x in xs)


def rand_qkv(B, H, N, d, dv, seed, dtype, scale_qk=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, N, d, generator=g) * scale_qk).to(dtype)
    k = (torch.randn(B, H, N, d, generator=g) * scale_qk).to(dtype)
    v = torch.randn(B, H, N, dv, generator=g).to(dtype)
    return q, k, v


def err(y, want):
    return ref.rel_err(y.detach().cpu(), want)


def rounded_err(y, want):
    """max |y - y_ref| / (|y_ref| + rms(y_ref)), for outputs rounded to bf16: BASED outputs of
    the first rows are an order of magnitude above the rms of the rest, so a max |error| / rms
    metric would mostly measure the output rounding of those rows."""
    y = y.detach().cpu().double()
    want = want.double()
    return ((y - want).abs() / (want.abs() + want.pow(2).mean().sqrt())).max().item()


def rows_fp64(q, k, v, b, h, rows, eps=1e-6, normalize=True):
    """Dense fp64 BASED output of the given query rows of head (b, h) over all earlier keys:
    the oracle for a few rows of a sequence too long for the dense t x t form."""
    import math
    qq, kk, vv = q[b, h].double(), k[b, h].double(), v[b, h].double()
    d = qq.shape[-1]
    s = (qq[rows] / math.sqrt(d)) @ kk.T
    mask = torch.arange(qq.shape[0]).unsqueeze(0) <= rows.unsqueeze(1)
    p = (1 + s + 0.5 * s * s) * mask
    num = p @ vv
    return num / (p.sum(-1, keepdim=True) + eps) if normalize else num


def head_errs(y, want):
    """Parity metric per (b, h) head: each head normalised by its own rms."""
    y = y.detach().cpu()
    return [ref.rel_err(y[b, h], want[b, h]) for b in range(y.shape[0]) for h in range(y.shape[1])]
