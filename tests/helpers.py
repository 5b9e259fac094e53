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
