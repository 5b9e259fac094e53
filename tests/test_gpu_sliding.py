"""GPU parity of the sliding-window softmax kernel (la_sliding_window_fwd) against the oracle."""

import math

import pytest
import torch

from oracle import reference as ref
from tests.helpers import err, load_golden, rand_qkv, to_dev

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
TOL_F32 = 1e-4


def _kernels():
    import kernels
    return kernels


@pytest.mark.parametrize("name", ["sliding_b1h2n131d64w1", "sliding_b1h2n131d64w17", "sliding_b1h2n131d64w64"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_golden(name, dtype):
    K = _kernels()
    g = load_golden(name)
    q, k, v = (torch.from_numpy(g[x]) for x in "qkv")
    y = K.sliding_window_attn(*to_dev(q, k, v, dtype=dtype), window_size=int(g["window"]), out_dtype=torch.float32)
    e = err(y, torch.from_numpy(g["y"]))
    print(f"{name} {dtype} err={e:.3e}")
    assert e < (TOL_BF16 if dtype == torch.bfloat16 else TOL_F32)


@pytest.mark.parametrize("W", [1, 2, 31, 32, 33, 63, 64, 65, 100, 128, 129, 300, 5000])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_windows(W, dtype):
    K = _kernels()
    q, k, v = rand_qkv(1, 2, 517, 64, 64, seed=W, dtype=dtype)
    y = K.sliding_window_attn(*to_dev(q, k, v), window_size=W, out_dtype=torch.float32)
    want = ref.sliding_dense(q, k, v, window_size=W)
    e = err(y, want)
    print(f"W={W} {dtype} err={e:.3e}")
    assert e < (TOL_BF16 if dtype == torch.bfloat16 else TOL_F32)


@pytest.mark.parametrize("d,dv", [(16, 16), (32, 64), (64, 32), (128, 128), (8, 24), (40, 72)])
def test_head_dims(d, dv):
    K = _kernels()
    q, k, v = rand_qkv(2, 1, 300, d, dv, seed=d + dv, dtype=torch.bfloat16)
    y = K.sliding_window_attn(*to_dev(q, k, v), window_size=50, out_dtype=torch.float32)
    want = ref.sliding_dense(q, k, v, window_size=50)
    assert err(y, want) < TOL_BF16


def test_window_one_is_identity():
    K = _kernels()
    q, k, v = to_dev(*rand_qkv(1, 2, 130, 64, 64, seed=1, dtype=torch.bfloat16))
    y = K.nki_sliding_window_attn(q, k, v, window_size=1)
    assert torch.equal(y, v)


def test_full_window_is_causal_sdpa():
    K = _kernels()
    q, k, v = rand_qkv(1, 2, 200, 64, 64, seed=5, dtype=torch.float32)
    y = K.nki_sliding_window_attn(*to_dev(q, k, v), window_size=10_000)
    want = torch.nn.functional.scaled_dot_product_attention(q.double(), k.double(), v.double(), is_causal=True)
    assert err(y, want) < TOL_F32


def test_sliding_w64_bf16_b2h16n4096():
    K = _kernels()
    cfg = ref.CONFIGS["sliding_w64_bf16_b2h16n4096"]
    q, k, v = ref.config_inputs(cfg)
    y = K.sliding_window_attn(*to_dev(q, k, v), window_size=cfg.window, out_dtype=torch.float32)
    want = ref.sliding_banded(q, k, v, window_size=cfg.window, dtype=torch.float64)
    e = err(y, want)
    print(f"sliding W64 B2 H16 N4096 err={e:.3e}")
    assert e < TOL_BF16
    y16 = K.nki_sliding_window_attn(*to_dev(q, k, v), window_size=cfg.window)
    assert y16.dtype == torch.bfloat16 and torch.equal(y16, y.to(torch.bfloat16))


@pytest.mark.parametrize("d,dv", [(16, 32), (16, 64), (32, 32), (32, 64), (64, 32), (64, 64)])
@pytest.mark.parametrize("W", [1, 37, 64, 65, 66, 100, 128, 129])
def test_resident_window_shapes(d, dv, W):
    """W <= 129 with d in {16, 32, 64} and dv in {32, 64} runs the LDS-resident kernel (one extra
    key block per tile above W = 65); ragged N so that the last 256-query tile and its key blocks
    are partial."""
    K = _kernels()
    q, k, v = rand_qkv(1, 3, 333, d, dv, seed=d * 7 + dv + W, dtype=torch.bfloat16)
    y = K.sliding_window_attn(*to_dev(q, k, v), window_size=W, out_dtype=torch.float32)
    want = ref.sliding_dense(q, k, v, window_size=W)
    assert err(y, want) < TOL_BF16


@pytest.mark.parametrize("W", [64, 65, 66, 128, 129])
def test_resident_matches_streaming_path(W):
    """The same inputs through the resident kernel (16-byte aligned output) and through the
    streaming kernel (fp32 output 4 bytes off 16-byte alignment, which the resident kernel
    requires), both through the C ABI."""
    from kernels import _lib
    L = _lib.lib()
    B, H, N, d, dv = 2, 2, 700, 64, 64
    q, k, v = to_dev(*rand_qkv(B, H, N, d, dv, seed=9 + W, dtype=torch.bfloat16))
    st = torch.cuda.current_stream().cuda_stream
    outs = []
    for off in (0, 1):
        buf = torch.empty(B * H * N * dv + 4, dtype=torch.float32, device="cuda")
        out = buf[off:off + B * H * N * dv].view(B, H, N, dv)
        assert (out.data_ptr() % 16 == 0) == (off == 0)
        assert L.la_sliding_window_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), 1, out.data_ptr(), 0, B, H, N, d, dv,
                                       W, 1.0 / math.sqrt(d), st) == 0
        outs.append(out.clone())
    want = ref.sliding_dense(q.cpu(), k.cpu(), v.cpu(), window_size=W)
    assert err(outs[0], want) < TOL_BF16 and err(outs[1], want) < TOL_BF16
    assert (outs[0] - outs[1]).abs().max().item() < 1e-3
