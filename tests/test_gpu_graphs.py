"""The kernels under HIP graph capture (torch.cuda.CUDAGraph): the library launches only kernels
on the caller's stream (no memset, allocation or synchronisation), so a captured call replays.
Each graph is replayed several times with eager work and synchronisations between the replays,
and every replay is checked against the eager result."""

import pytest
import torch

from tests.helpers import rand_qkv, to_dev

pytestmark = pytest.mark.gpu


def _kernels():
    import kernels
    return kernels


def _capture(fn):
    """Warm up on a side stream (default priority), then capture fn() into a graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def _eager_noise(K):
    q, k, v = to_dev(*rand_qkv(1, 2, 200, 16, 32, seed=77, dtype=torch.bfloat16))
    K.sliding_window_attn(q, k, v, window_size=33)
    torch.cuda.synchronize()


@pytest.mark.parametrize("N", [300, 2048])
def test_parallel_forward_replays(N):
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(1, 4, N, 16, 64, seed=N, dtype=torch.bfloat16, scale_qk=0.5))
    want = K.solution_nki(q, k, v)
    g, y = _capture(lambda: K.solution_nki(q, k, v))
    for _ in range(3):
        _eager_noise(K)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want)


def test_chunked_prefill_with_state_replays():
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(2, 2, 600, 16, 64, seed=3, dtype=torch.bfloat16, scale_qk=0.5))
    _, st0 = K.based_chunked(q[:, :, :200], k[:, :, :200], v[:, :, :200], return_state=True)
    args = (q[:, :, 200:], k[:, :, 200:], v[:, :, 200:])
    want, want_st = K.based_chunked(*args, return_state=True, state_in=st0, prev_tokens=200)
    g, (y, st) = _capture(lambda: K.based_chunked(*args, return_state=True, state_in=st0, prev_tokens=200))
    for _ in range(3):
        _eager_noise(K)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want) and torch.equal(st, want_st)


def test_decode_step_replays():
    """A decode step updates its state in place: the state is reset from a copy (eagerly) before
    every replay, and each replay must reproduce the eager step."""
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(2, 16, 1, 16, 64, seed=5, dtype=torch.bfloat16))
    base = torch.randn(2, 16, K.feature_dim(16), 65, device="cuda").abs()
    st_eager = base.clone()
    want = K.based_decode_step(q, k, v, st_eager)
    st = base.clone()
    g, y = _capture(lambda: K.based_decode_step(q, k, v, st))
    for _ in range(3):
        _eager_noise(K)
        st.copy_(base)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want) and torch.equal(st, st_eager)


def test_sliding_identity_and_layer_replay():
    """Sliding-window (resident and streaming windows), identity-map and full-layer calls captured
    together in one graph; every replay matches the eager calls bit for bit."""
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(2, 2, 700, 64, 64, seed=11, dtype=torch.bfloat16, scale_qk=0.5))
    q16, k16 = to_dev(*rand_qkv(2, 2, 700, 16, 1, seed=12, dtype=torch.bfloat16, scale_qk=0.5))[:2]

    def calls():
        return (K.sliding_window_attn(q, k, v, window_size=64),
                K.sliding_window_attn(q, k, v, window_size=300),
                K.identity_linear_attn(q16, k16, v),
                K.based_layer_attn(q16, k16, v, window_size=64, q_sw=q, k_sw=k))

    want = calls()
    g, outs = _capture(calls)
    for _ in range(3):
        _eager_noise(K)
        g.replay()
        torch.cuda.synchronize()
        for y, w in zip(outs, want):
            assert torch.equal(y, w)
