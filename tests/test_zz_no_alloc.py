"""The no-allocation chunked entry point (la_based_chunked_fwd_noalloc) against la_based_chunked_fwd
through the C ABI: two calls in a row on one device, the second with a smaller input, each bit
for bit equal to the workspace entry point's output and exported state (the same kernels run on
the same inputs; only the scratch memory differs) -- for the d = 16 recurrence and for shapes of
the segment-state path (d = 64 bf16, fp32 inputs) whose scratch fits the fixed array."""

import os
import sys

import pytest
import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from helpers import rand_qkv  # noqa: E402

pytestmark = pytest.mark.gpu

F = 153


def _workspace_call(L, q, k, v, out, state, chunk):
    B, H, N, d = q.shape
    dv = v.shape[-1]
    nb = int(L.la_based_chunked_workspace_bytes(B, H, N, d, dv, chunk))
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=q.device)
    stream = torch.cuda.current_stream().cuda_stream
    return L.la_based_chunked_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), 1, out.data_ptr(), 0, B, H, N, d, dv,
                                  chunk, 0.25, 1e-6, 1, ws.data_ptr(), nb, state.data_ptr(), stream)


def _noalloc_call(L, q, k, v, out, state, chunk):
    B, H, N, d = q.shape
    dv = v.shape[-1]
    stream = torch.cuda.current_stream().cuda_stream
    return L.la_based_chunked_fwd_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), 1, out.data_ptr(), 0, B, H, N, d,
                                          dv, chunk, 0.25, 1e-6, 1, state.data_ptr(), stream)


@pytest.mark.parametrize("shapes", [((2, 16, 8192, 64), (1, 4, 3000, 48)), ((1, 16, 65536, 64), (2, 8, 700, 64))])
def test_noalloc_matches_workspace_entry_point(shapes):
    from kernels import _lib
    L = _lib.lib()
    for i, (B, H, N, dv) in enumerate(shapes):
        print(f"noalloc call {i}: B{B} H{H} N{N} dv{dv}", flush=True)
        q, k, v = (x.cuda() for x in rand_qkv(B, H, N, 16, dv, 40 + i, torch.bfloat16, scale_qk=0.5))
        want = torch.empty(B, H, N, dv, dtype=torch.float32, device="cuda")
        want_s = torch.empty(B, H, F, dv + 1, dtype=torch.float32, device="cuda")
        got = torch.full_like(want, float("nan"))
        got_s = torch.full_like(want_s, float("nan"))
        assert _workspace_call(L, q, k, v, want, want_s, 64) == 0
        assert _noalloc_call(L, q, k, v, got, got_s, 64) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, want), (got - want).abs().max().item()
        assert torch.equal(got_s, want_s), (got_s - want_s).abs().max().item()


def _general_pair(L, dt, B, H, N, d, dv, seed):
    torch_dt = torch.bfloat16 if dt == 1 else torch.float32
    q, k, v = (x.cuda() for x in rand_qkv(B, H, N, d, dv, seed, torch_dt, scale_qk=0.5))
    stream = torch.cuda.current_stream().cuda_stream
    nb = int(L.la_based_chunked_workspace_bytes_dt(B, H, N, d, dv, 64, dt))
    assert 0 < nb <= (32 << 20), nb
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    want = torch.empty(B, H, N, dv, dtype=torch.float32, device="cuda")
    got = torch.full_like(want, float("nan"))
    scale = 1.0 / d ** 0.5
    assert L.la_based_chunked_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), dt, want.data_ptr(), 0, B, H, N, d, dv,
                                  64, scale, 1e-6, 1, ws.data_ptr(), nb, None, stream) == 0
    assert L.la_based_chunked_fwd_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), dt, got.data_ptr(), 0, B, H, N,
                                          d, dv, 64, scale, 1e-6, 1, None, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(got, want), (got - want).abs().max().item()


@pytest.mark.parametrize("dt,shapes", [(1, ((1, 4, 3000, 64, 64), (1, 2, 1100, 64, 48))),
                                       (0, ((2, 4, 3000, 16, 64), (1, 3, 1200, 16, 32)))])
def test_noalloc_segment_state_path(dt, shapes):
    from kernels import _lib
    L = _lib.lib()
    for i, (B, H, N, d, dv) in enumerate(shapes):
        print(f"noalloc segment-state call {i}: dtype {dt} B{B} H{H} N{N} d{d} dv{dv}", flush=True)
        _general_pair(L, dt, B, H, N, d, dv, 50 + i)
