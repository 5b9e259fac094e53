"""GPU parity of the decode step (la_based_decode_step): one token per head on the state the
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
