"""GPU parity of the Taylor feature map kernel (la_taylor_feature_map)."""

import pytest
import torch

from oracle import reference as ref
from tests.helpers import load_golden

pytestmark = pytest.mark.gpu


def _kernels():
    import kernels
    return kernels


@pytest.mark.parametrize("name", ["phi_d4", "phi_d16"])
def test_golden(name):
    K = _kernels()
    g = load_golden(name)
    x = torch.from_numpy(g["x"])
    y = K.taylor_feature_map(x.cuda()).cpu()
    assert y.dtype == torch.float32
    assert torch.allclose(y.double(), torch.from_numpy(g["phi"]), rtol=2e-7, atol=1e-7)


@pytest.mark.parametrize("d", [1, 2, 3, 5, 16, 17, 64, 128])
def test_matches_reference_fp32(d):
    K = _kernels()
    x = torch.randn(3, 7, d)
    y = K.taylor_feature_map(x.cuda()).cpu()
    want = ref.taylor_feature_map(x)
    assert y.shape == want.shape
    ulp = torch.finfo(torch.float32).eps * want.abs().clamp_min(1e-30)
    print(f"d={d} exact={torch.equal(y, want)} max_ulp={((y - want).abs() / ulp).max().item():.2f}")
    assert ((y - want).abs() <= ulp).all()


def test_bf16_input():
    K = _kernels()
    x = torch.randn(50, 16).to(torch.bfloat16)
    y = K.taylor_feature_map(x.cuda()).cpu()
    assert y.dtype == torch.bfloat16
    want = ref.taylor_feature_map(x.double())
    assert torch.allclose(y.double(), want, rtol=8e-3, atol=1e-6)
