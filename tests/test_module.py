"""The module-level callers (reference benchmarks/based_attention_benchmark.py:24-69): parameter
names and shapes (CPU), and on the GPU the layer's output against the same layer composed from
the oracle (projections and the dense BASED attention in fp64 on the same rounded operands)."""

import math

import pytest
import torch

from oracle import reference as ref
from tests.helpers import err, rounded_err


def _modules():
    import kernels
    return kernels


def _oracle_layer(mod, x):
    """The layer on the CPU: q/k/v projections rounded to the module's dtype, attention in fp64 by
    the oracle (kernels/pytorch_attention.py:27-42), heads merged, rounded, o_proj in fp64."""
    dt = x.dtype
    xs = x.detach().cpu().double()
    W = {n: getattr(mod, n).weight.detach().cpu().double() for n in ("q_proj", "k_proj", "v_proj", "o_proj")}
    b, t, dim = xs.shape
    h, hd = mod.num_heads, mod.head_dim
    heads = [(xs @ W[n].T).to(dt).view(b, t, h, hd).transpose(1, 2) for n in ("q_proj", "k_proj", "v_proj")]
    y, _, _ = ref.based_dense(*heads, eps=mod.eps)
    y = y.transpose(1, 2).reshape(b, t, dim).to(dt).double()
    return y @ W["o_proj"].T


def test_parameter_names_and_shapes():
    K = _modules()
    for cls in (K.TrainiumBasedLinearAttention, K.TrainiumBasedLinearAttentionNKI):
        m = cls(256, heads=16)
        assert (m.num_heads, m.head_dim, m.eps) == (16, 16, 1e-6)
        sd = m.state_dict()
        assert sorted(sd) == ["k_proj.weight", "o_proj.weight", "q_proj.weight", "v_proj.weight"]
        assert all(w.shape == (256, 256) for w in sd.values())
    with pytest.raises(AssertionError):
        K.TrainiumBasedLinearAttentionNKI(100, heads=8)
    with pytest.raises(ValueError):
        K.TrainiumBasedLinearAttentionNKI(64, heads=4, dispatch="pytorch")


def test_no_host_path():
    K = _modules()
    m = K.TrainiumBasedLinearAttentionNKI(64, heads=4)
    with pytest.raises(RuntimeError):
        m(torch.randn(1, 8, 64))   # CPU tensors: the kernels run on the GPU only


@pytest.mark.gpu
@pytest.mark.parametrize("cls,dim,heads,t,dtype", [
    ("TrainiumBasedLinearAttentionNKI", 256, 16, 300, torch.bfloat16),
    ("TrainiumBasedLinearAttention", 256, 16, 300, torch.bfloat16),    # chunked kernel (t >= 256)
    ("TrainiumBasedLinearAttention", 256, 16, 100, torch.bfloat16),    # fused kernel (t < 256)
    ("TrainiumBasedLinearAttentionNKI", 128, 8, 129, torch.float32),
    ("TrainiumBasedLinearAttentionNKI", 512, 8, 200, torch.bfloat16),  # head_dim 64
])
def test_layer_matches_oracle(cls, dim, heads, t, dtype):
    K = _modules()
    torch.manual_seed(dim + t)
    m = getattr(K, cls)(dim, heads=heads).to(device="cuda", dtype=dtype)
    x = (torch.randn(2, t, dim) / math.sqrt(dim) * 4).to(dtype).cuda()
    with torch.no_grad():
        y = m(x)
    assert y.shape == x.shape and y.dtype == dtype
    want = _oracle_layer(m, x)
    if dtype == torch.bfloat16:
        assert rounded_err(y, want) < 2e-2   # rounded twice: attention output, then o_proj
    else:
        assert err(y, want) < 1e-4


@pytest.mark.gpu
def test_reference_state_dict_loads_and_weight_changes_take_effect():
    K = _modules()
    torch.manual_seed(1)
    src = torch.nn.ModuleDict({n: torch.nn.Linear(128, 128, bias=False) for n in ("q_proj", "k_proj", "v_proj",
                                                                                    "o_proj")})
    m = K.TrainiumBasedLinearAttentionNKI(128, heads=8).cuda()
    m.load_state_dict({f"{n}.weight": src[n].weight.detach() for n in src})
    x = torch.randn(1, 70, 128).cuda() * 0.3
    with torch.no_grad():
        y0 = m(x)
        assert err(y0, _oracle_layer(m, x)) < 1e-4
        m.k_proj.weight.mul_(0.5)                 # in place: the cached q/k/v weight is rebuilt
        y1 = m(x)
    assert not torch.equal(y0, y1)
    assert err(y1, _oracle_layer(m, x)) < 1e-4


@pytest.mark.gpu
def test_backward_raises():
    K = _modules()
    m = K.TrainiumBasedLinearAttentionNKI(64, heads=4).cuda()
    x = torch.randn(1, 16, 64, device="cuda", requires_grad=True)
    y = m(x)
    with pytest.raises(RuntimeError, match="forward-only"):
        y.sum().backward()
