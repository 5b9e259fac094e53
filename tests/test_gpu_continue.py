"""GPU parity of the chunked kernel continued from a state (la_based_chunked_fwd_continue):
a sequence processed in pieces -- each piece starting from the previous piece's exported state
-- against the fp64 oracle of the whole sequence (dense BASED rows, the state's closed form)."""

import pytest
import torch

from oracle import reference as ref
from tests.helpers import err, rand_qkv, to_dev

pytestmark = pytest.mark.gpu


def _kernels():
    import kernels
    return kernels


def _state_closed_form(k, v):
    phik = ref.taylor_feature_map(k.double())
    return torch.cat([phik.transpose(-2, -1) @ v.double(), phik.sum(-2).unsqueeze(-1)], dim=-1)


@pytest.mark.parametrize("B,H,pieces,dv", [(2, 3, (300, 400), 64), (1, 2, (129, 1, 5, 250), 32),
                                           (2, 16, (1000, 1000), 64)])
def test_pieces_equal_whole(B, H, pieces, dv):
    K = _kernels()
    T = sum(pieces)
    q, k, v = rand_qkv(B, H, T, 16, dv, seed=T + dv, dtype=torch.bfloat16, scale_qk=0.6)
    qd, kd, vd = to_dev(q, k, v)
    st, t0, ys = None, 0, []
    for n in pieces:
        sl = slice(t0, t0 + n)
        if st is None:
            y, st = K.based_chunked(qd[:, :, sl], kd[:, :, sl], vd[:, :, sl], out_dtype=torch.float32,
                                    return_state=True)
        else:
            y, st = K.based_chunked(qd[:, :, sl], kd[:, :, sl], vd[:, :, sl], out_dtype=torch.float32,
                                    return_state=True, state_in=st)
        ys.append(y)
        t0 += n
    want, _, _ = ref.based_dense(q, k, v)
    assert err(torch.cat(ys, dim=2), want) < 2e-2
    assert ref.rel_err(st.cpu(), _state_closed_form(k, v)) < 1e-2


def test_zero_state_is_a_plain_call():
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(2, 2, 777, 16, 64, seed=5, dtype=torch.bfloat16, scale_qk=0.6))
    y0, s0 = K.based_chunked(q, k, v, out_dtype=torch.float32, return_state=True)
    zero = torch.zeros_like(s0)
    y1, s1 = K.based_chunked(q, k, v, out_dtype=torch.float32, return_state=True, state_in=zero, prev_tokens=0)
    assert torch.equal(y0, y1) and torch.equal(s0, s1)
    assert torch.equal(zero, torch.zeros_like(zero))      # state_in is read, not written


def test_prefill_decode_continue():
    """Prefill, three decode steps on the exported state, then a chunked continuation from the
    decode-updated state: all outputs are rows of dense BASED over the whole sequence."""
    K = _kernels()
    B, H, n1, n2, n3 = 1, 4, 200, 3, 150
    T = n1 + n2 + n3
    q, k, v = rand_qkv(B, H, T, 16, 64, seed=11, dtype=torch.bfloat16, scale_qk=0.6)
    qd, kd, vd = to_dev(q, k, v)
    y1, st = K.based_chunked(qd[:, :, :n1], kd[:, :, :n1], vd[:, :, :n1], out_dtype=torch.float32,
                             return_state=True)
    y2 = [K.based_decode_step(qd[:, :, t], kd[:, :, t], vd[:, :, t], st).float() for t in range(n1, n1 + n2)]
    y3 = K.based_chunked(qd[:, :, n1 + n2:], kd[:, :, n1 + n2:], vd[:, :, n1 + n2:], out_dtype=torch.float32,
                         state_in=st)
    want, _, _ = ref.based_dense(q, k, v)
    assert err(y1, want[:, :, :n1]) < 2e-2
    assert err(torch.stack(y2, dim=2), want[:, :, n1:n1 + n2]) < 2e-2
    assert err(y3, want[:, :, n1 + n2:]) < 2e-2


def test_long_prefix_spot_rows():
    """A 60000-token prefix carried as a state into a 2000-token piece (the fp16 range scaling is
    chosen from the total length): rows of the piece against fp64 prefix states."""
    K = _kernels()
    B, H, n1, n2 = 1, 2, 60000, 2000
    q, k, v = rand_qkv(B, H, n1 + n2, 16, 64, seed=13, dtype=torch.bfloat16, scale_qk=0.5)
    qd, kd, vd = to_dev(q, k, v)
    _, st = K.based_chunked(qd[:, :, :n1], kd[:, :, :n1], vd[:, :, :n1], return_state=True)
    y = K.based_chunked(qd[:, :, n1:], kd[:, :, n1:], vd[:, :, n1:], out_dtype=torch.float32, state_in=st).cpu()
    for h in range(H):
        phik = ref.taylor_feature_map(k[0, h].double())
        vv = v[0, h].double()
        for t in [0, 1, 127, 128, 1999]:
            u = n1 + t
            S = phik[: u + 1].T @ vv[: u + 1]
            z = phik[: u + 1].sum(0)
            phq = ref.taylor_feature_map(q[0, h, u].double())
            want = (phq @ S) / (phq @ z + 1e-6)
            got = y[0, h, t].double()
            assert (got - want).abs().max() / want.pow(2).mean().sqrt() < 2e-2, (h, t)


def test_continue_errors():
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(1, 1, 8, 16, 64, seed=0, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError):
        K.based_chunked(q, k, v, state_in=torch.zeros(1, 1, 153, 64, device="cuda"))   # width
    q2, k2, v2 = to_dev(*rand_qkv(1, 1, 8, 32, 64, seed=0, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError):
        K.based_chunked(q2, k2, v2, state_in=torch.zeros(1, 1, 153, 65, device="cuda"))   # d = 32 has 561 features
    q3, k3, v3 = to_dev(*rand_qkv(1, 1, 8, 80, 64, seed=0, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError):
        K.based_chunked(q3, k3, v3, state_in=torch.zeros(1, 1, 3321, 65, device="cuda"))  # d = 80: no chunked path
