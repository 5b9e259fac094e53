"""GPU parity of the decode step (la_based_decode_step{,_ws}): one token per head on the state the
chunked kernel exports, against the fp64 oracle (dense BASED over the whole sequence, and the
state's closed form sum_u phi(k_u) [v_u | 1])."""

import pytest
import torch

from oracle import reference as ref
from tests.helpers import err, rand_qkv, rounded_err, to_dev

pytestmark = pytest.mark.gpu


def _kernels():
    import kernels
    return kernels


def _state_closed_form(k, v):
    phik = ref.taylor_feature_map(k.double())
    return torch.cat([phik.transpose(-2, -1) @ v.double(), phik.sum(-2).unsqueeze(-1)], dim=-1)


@pytest.mark.parametrize("B,H,N,M,dv", [(2, 3, 300, 6, 64), (1, 2, 129, 4, 24)])
def test_prefill_then_decode(B, H, N, M, dv):
    """Prefill N tokens with the chunked kernel (state exported), then M decode steps: every
    step's output equals the dense BASED row of the full sequence, and the final state the
    closed form of all N + M tokens."""
    K = _kernels()
    q, k, v = rand_qkv(B, H, N + M, 16, dv, seed=N + M, dtype=torch.bfloat16, scale_qk=0.6)
    qd, kd, vd = to_dev(q, k, v)
    _, st = K.based_chunked(qd[:, :, :N], kd[:, :, :N], vd[:, :, :N], out_dtype=torch.float32,
                            return_state=True)
    ys = [K.based_decode_step(qd[:, :, t:t + 1], kd[:, :, t:t + 1], vd[:, :, t:t + 1], st) for t in range(N, N + M)]
    y = torch.cat(ys, dim=2)
    assert y.shape == (B, H, M, dv) and y.dtype == torch.bfloat16
    want, _, _ = ref.based_dense(q, k, v)
    assert rounded_err(y, want[:, :, N:]) < 2e-2
    assert ref.rel_err(st.cpu(), _state_closed_form(k, v)) < 1e-2


@pytest.mark.parametrize("d,dv", [(16, 8), (4, 3), (64, 128), (1, 1)])
def test_decode_from_empty_state_fp32(d, dv):
    """From a zero state, decoding a whole sequence token by token is dense BASED (fp32 bar) and
    leaves the state's closed form; normalize=False returns the numerator."""
    K = _kernels()
    B, H, N = 2, 2, 20
    q, k, v = rand_qkv(B, H, N, d, dv, seed=d * 10 + dv, dtype=torch.float32, scale_qk=0.5)
    qd, kd, vd = to_dev(q, k, v)
    F = K.feature_dim(d)
    st = torch.zeros(B, H, F, dv + 1, device="cuda")
    st_num = torch.zeros_like(st)
    ys, nums = [], []
    for t in range(N):
        ys.append(K.based_decode_step(qd[:, :, t], kd[:, :, t], vd[:, :, t], st))
        nums.append(K.based_decode_step(qd[:, :, t], kd[:, :, t], vd[:, :, t], st_num, normalize=False))
    y = torch.stack(ys, dim=2)
    num = torch.stack(nums, dim=2)
    want, want_num, _ = ref.based_dense(q, k, v)
    assert err(y, want) < 1e-4
    assert err(num, want_num) < 1e-4
    assert ref.rel_err(st.cpu(), _state_closed_form(k, v)) < 1e-5
    assert torch.equal(st, st_num)


def test_decode_errors():
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(1, 2, 1, 16, 8, seed=0, dtype=torch.bfloat16))
    good = torch.zeros(1, 2, K.feature_dim(16), 9, device="cuda")
    with pytest.raises(RuntimeError):
        K.based_decode_step(q, k, v, good[..., :8].contiguous())           # wrong state width
    with pytest.raises(RuntimeError):
        K.based_decode_step(q, k, v, good.double())                        # fp64 state
    q2, k2, v2 = to_dev(*rand_qkv(1, 2, 2, 16, 8, seed=0, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError):
        K.based_decode_step(q2, k2, v2, good)                              # two tokens
    q3 = torch.zeros(1, 2, 65, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        K.based_decode_step(q3, q3, v[:, :, 0], torch.zeros(1, 2, K.feature_dim(65), 9, device="cuda"))   # d > 64


@pytest.mark.parametrize("B,H,d,dv", [(2, 16, 16, 128), (40, 16, 16, 128), (1, 1, 16, 66), (1, 3, 64, 128),
                                      (8, 16, 32, 64), (2, 16, 16, 64), (64, 16, 16, 64), (3, 5, 7, 5),
                                      (1, 1, 1, 1)])
def test_split_rows_match_one_group_per_head(B, H, d, dv):
    """la_based_decode_step_ws (state rows split over work-groups when the batch is small and the
    state does not fit in LDS) against la_based_decode_step, through the C ABI: the updated states are
    bit-identical (the same fma per element) and the outputs agree to fp32 rounding (the partial
    column sums are added in another order: the fp32 bar); twice in a row on the same workspace."""
    K = _kernels()
    from kernels import _lib
    L = _lib.lib()
    F = K.feature_dim(d)
    need = int(L.la_based_decode_workspace_bytes(B, H, d, dv))
    assert (need > 0) == (B * H < 1024 and F > 8 and F * (dv + 1) > 10240)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    # the state of 8 earlier tokens (every token adds 1 + s + s^2/2 >= 1/2 to a denominator)
    _, k0, v0 = rand_qkv(B, H, 8, d, dv, seed=B * 1000 + d * 10 + dv, dtype=torch.float32, scale_qk=0.5)
    st = _state_closed_form(k0, v0).float().cuda()
    assert st.shape == (B, H, F, dv + 1)
    st_one, st_split = st.clone(), st.clone()
    for step in range(2):
        q, k, v = to_dev(*rand_qkv(B, H, 1, d, dv, seed=step + 7 * d, dtype=torch.float32, scale_qk=0.5))
        y_one = torch.empty(B, H, dv, device="cuda")
        y_split = torch.full((B, H, dv), float("nan"), device="cuda")
        args = (_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), 0)
        rc = L.la_based_decode_step(*args, _lib.ptr(st_one), _lib.ptr(y_one), 0, B, H, d, dv, 1e-6, 1,
                                    _lib.stream_of(q))
        assert rc == 0
        rc = L.la_based_decode_step_ws(*args, _lib.ptr(st_split), _lib.ptr(y_split), 0, B, H, d, dv, 1e-6, 1,
                                       _lib.ptr(ws), need, _lib.stream_of(q))
        assert rc == 0
        torch.cuda.synchronize()
        assert torch.equal(st_one, st_split)
        assert err(y_split, y_one.cpu()) < 1e-4   # the fp32 bar (2145-term sums at d = 64)
