"""CPU checks of the C ABI: the library loads, exports every entry point include/based_la.h
declares, and rejects bad arguments on the host before any launch (no GPU needed)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "based_la.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(la_\w+)\s*\(", text, re.M)))


def _lib():
    from kernels import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libbased_la.so not built")
    return _lib.lib()


def test_header_declares_expected_entry_points():
    assert _declared() == sorted([
        "la_abi_version", "la_status_string", "la_based_parallel_workspace_bytes", "la_based_parallel_fwd",
        "la_based_parallel_pack", "la_based_parallel_fwd_packed", "la_based_chunked_workspace_bytes",
        "la_based_chunked_workspace_bytes_dt", "la_based_chunked_chunk_used", "la_based_chunked_fwd",
        "la_based_chunked_fwd_continue", "la_based_chunked_fwd_noalloc", "la_based_chunked_fwd_num_den",
        "la_sliding_window_fwd",
        "la_sliding_window_fwd_add", "la_based_layer_fwd", "la_based_decode_step", "la_based_decode_workspace_bytes",
        "la_based_decode_step_ws", "la_identity_workspace_bytes", "la_identity_linear_fwd",
        "la_taylor_feature_map"])


def test_library_exports_every_declared_symbol():
    lib = _lib()
    for name in _declared():
        assert hasattr(lib, name), name


def test_abi_version_and_status_strings():
    lib = _lib()
    assert lib.la_abi_version() == 10
    for code in range(-10, 1):
        s = lib.la_status_string(code).decode()
        assert s and s != "unknown status"


def _codes():
    from kernels import _lib
    return _lib


P = ctypes.c_void_p(16)   # dummy non-null, 16-byte aligned pointer; never dereferenced on error paths


def test_parallel_argument_errors():
    lib = _lib()
    f = lib.la_based_parallel_fwd
    need = lib.la_based_parallel_workspace_bytes(1, 1, 8, 16, 64, 1)
    ok_args = dict(q=P, k=P, v=P, dt=1, out=P, odt=1, den=None, B=1, H=1, N=8, d=16, dv=64, scale=0.25, eps=1e-6,
                   norm=1, ws=P, ws_bytes=need)

    def call(**kw):
        a = dict(ok_args, **kw)
        return f(a["q"], a["k"], a["v"], a["dt"], a["out"], a["odt"], a["den"], a["B"], a["H"], a["N"], a["d"],
                 a["dv"], a["scale"], a["eps"], a["norm"], a["ws"], a["ws_bytes"], None)

    assert call(q=None) == -1
    assert call(d=0) == -2
    assert call(N=-1) == -2
    assert call(dt=7) == -3
    assert call(odt=2) == -3
    assert call(scale=0.0) == -4
    assert call(scale=float("nan")) == -4
    assert call(eps=-1.0) == -4
    assert call(d=129) == -5
    assert call(dv=200) == -5
    assert call(q=ctypes.c_void_p(17)) == -8
    assert call(ws=None) == -6                 # bf16, d = 16, dv = 64 needs the V^T workspace
    assert call(ws_bytes=need - 1) == -6
    assert call(ws=ctypes.c_void_p(24)) == -8
    assert call(N=0) == 0          # empty: nothing to launch
    assert call(B=0) == 0
    need32 = lib.la_based_parallel_workspace_bytes(1, 1, 8, 32, 64, 1)
    assert call(d=32, ws=None, ws_bytes=0) == -6      # bf16 register-staged shapes need the |v| maxima
    assert call(d=32, ws_bytes=need32 - 4) == -6
    assert call(dt=0, odt=0, ws=None, ws_bytes=0, q=ctypes.c_void_p(1 << 20), k=ctypes.c_void_p(1 << 21),
                v=ctypes.c_void_p(1 << 22), out=ctypes.c_void_p(1 << 23), N=0) == 0   # fp32: no workspace


def test_sliding_add_argument_errors():
    lib = _lib()
    f = lib.la_sliding_window_fwd_add
    ok = [P, P, P, 1, P, P, 1, 1, 1, 8, 16, 64, 64, 0.25, None]

    def call(i, x):
        a = list(ok)
        a[i] = x
        return f(*a)

    assert call(4, None) == -1                     # addend required
    assert call(4, ctypes.c_void_p(8)) == -8       # addend not 16-byte aligned
    assert call(0, None) == -1
    assert call(12, 0) == -4                       # window
    assert call(10, 129) == -5                     # d
    assert call(9, 0) == 0                         # N = 0: nothing to launch


def test_layer_argument_errors():
    """la_based_layer_fwd rejects what its kernel does not take before anything is launched."""
    lib = _lib()
    f = lib.la_based_layer_fwd
    need = lib.la_based_chunked_workspace_bytes(1, 1, 8, 16, 64, 64)
    W = ctypes.c_void_p(1 << 24)
    # q, k, v, q_sw, k_sw, dtype, out, out_dtype, B, H, N, d, dv, d_sw, window, scale, scale_sw, eps, ws, bytes, stream
    ok = [P, P, P, P, P, 1, P, 1, 1, 1, 8, 16, 64, 64, 64, 0.25, 0.125, 1e-6, W, need, None]

    def call(i, x):
        a = list(ok)
        a[i] = x
        return f(*a)

    assert call(3, None) == -1                     # q_sw
    assert call(4, None) == -1                     # k_sw
    assert call(5, 0) == -3                        # fp32 inputs: the two-launch layer
    assert call(11, 32) == -5                      # d != 16
    assert call(12, 72) == -5                      # dv > 64
    assert call(12, 20) == -5                      # dv % 8 != 0
    assert call(13, 48) == -5                      # d_sw not 16, 32 or 64
    assert call(14, 65) == -5                      # window > 64
    assert call(14, 0) == -5                       # window < 1
    assert call(16, 0.0) == -4                     # scale_sw
    assert call(3, ctypes.c_void_p((1 << 20) + 8)) == -8   # q_sw not 16-byte aligned
    assert call(10, 0) == 0                        # N = 0: nothing to launch


def test_chunked_continue_argument_errors():
    lib = _lib()
    f = lib.la_based_chunked_fwd_continue
    need = lib.la_based_chunked_workspace_bytes(1, 1, 8, 16, 64, 64)
    S = ctypes.c_void_p(1 << 20)
    ok = [P, P, P, 1, P, 1, 1, 1, 8, 16, 64, 64, 0.25, 1e-6, 1, P, need, S, 100, None, None]

    def call(i, x):
        a = list(ok)
        a[i] = x
        return f(*a)

    assert call(17, None) == -1                                   # state_in required
    assert call(17, ctypes.c_void_p((1 << 20) + 2)) == -8         # not 4-byte aligned
    assert call(18, -1) == -4                                     # prev_tokens
    assert call(19, ctypes.c_void_p((1 << 20) + 4096)) == -9      # state_out overlaps state_in
    assert call(15, ctypes.c_void_p((1 << 22) + 8)) == -8         # workspace not 16-byte aligned
    assert call(8, 0) == 0                                        # N = 0


def test_chunked_num_den_argument_errors():
    lib = _lib()
    f = lib.la_based_chunked_fwd_num_den
    need = lib.la_based_chunked_workspace_bytes(1, 1, 8, 16, 64, 64)
    D = ctypes.c_void_p(1 << 21)
    ok = [P, P, P, 1, P, D, 1, 1, 8, 16, 64, 64, 0.25, P, need, None]

    def call(i, x):
        a = list(ok)
        a[i] = x
        return f(*a)

    assert call(5, None) == -1                                    # den_out required
    assert call(5, ctypes.c_void_p((1 << 21) + 2)) == -8          # den_out not 4-byte aligned
    assert call(4, None) == -1                                    # num_out
    assert call(12, 0.0) == -4                                    # scale
    assert call(11, 0) == -2                                      # chunk
    assert call(9, 80) == -5                                      # d > 64
    need64 = lib.la_based_chunked_workspace_bytes_dt(1, 1, 2000, 64, 64, 64, 1)
    assert need64 > 0
    a = list(ok)
    a[8], a[9], a[14] = 2000, 64, need64 - 1
    assert f(*a) == -6                                            # workspace too small
    assert call(8, 0) == 0                                        # N = 0


def test_decode_argument_errors():
    lib = _lib()
    f = lib.la_based_decode_step
    ok = [P, P, P, 1, P, P, 1, 1, 2, 16, 64, 1e-6, 1, None]

    def call(i, x):
        a = list(ok)
        a[i] = x
        return f(*a)

    assert call(4, None) == -1                        # state
    assert call(4, ctypes.c_void_p(18)) == -8         # state not 4-byte aligned
    assert call(9, 65) == -5                          # d
    assert call(10, 129) == -5                        # dv
    assert call(11, -1.0) == -4                       # eps
    assert call(3, 5) == -3                           # dtype
    assert call(7, 0) == 0                            # B = 0: nothing to launch


def test_decode_workspace_sizes_and_errors():
    lib = _lib()
    ws = lib.la_based_decode_workspace_bytes
    # A head's state of F (dv + 1) <= 10240 floats is held in LDS by one work-group: no
    # workspace (d = 16: F = 153, so dv <= 65).  Larger states: B*H heads split into R row
    # groups of the F rows until about 1024 work-groups launch, at least 8 rows each: R = 20 for
    # 2 heads, 8 for 128, 2 for 640, 1 for 1024 (no workspace); one fp32 partial sum per group
    # and column (dv + 1 columns).
    assert ws(1, 2, 16, 64) == 0 and ws(1, 1, 16, 65) == 0 and ws(1, 1, 4, 128) == 0
    assert ws(1, 1, 16, 66) == 20 * 67 * 4
    assert ws(1, 2, 16, 128) == 2 * 20 * 129 * 4
    assert ws(8, 16, 16, 128) == 128 * 8 * 129 * 4
    assert ws(40, 16, 16, 128) == 640 * 2 * 129 * 4
    assert ws(64, 16, 16, 128) == 0
    assert ws(1, 1, 64, 128) == 269 * 129 * 4        # F = 2145 in groups of 8 rows
    assert ws(1, 1, 65, 8) == 0 and ws(1, 1, 16, 129) == 0 and ws(-1, 1, 16, 8) == 0
    f = lib.la_based_decode_step_ws
    need = ws(1, 2, 16, 128)
    ok = [P, P, P, 1, P, P, 1, 1, 2, 16, 128, 1e-6, 1, P, need, None]

    def call(i, x):
        a = list(ok)
        a[i] = x
        return f(*a)

    assert call(13, None) == -6                       # workspace needed
    assert call(14, need - 1) == -6                   # workspace too small
    assert call(13, ctypes.c_void_p((1 << 20) + 2)) == -8   # workspace not 4-byte aligned
    assert call(4, None) == -1                        # state
    assert call(9, 65) == -5                          # d
    assert call(11, float("nan")) == -4               # eps
    assert call(7, 0) == 0                            # B = 0: nothing to launch


def test_identity_workspace_and_argument_errors():
    lib = _lib()
    ws = lib.la_identity_workspace_bytes
    # one fp32 (dv x d) record per 256-token span of every head
    assert ws(2, 16, 8192, 16, 64) == 32 * 32 * 64 * 16 * 4
    assert ws(1, 1, 257, 64, 32) == 2 * 32 * 64 * 4
    assert ws(1, 1, 64, 48, 64) == 0 and ws(1, 1, 64, 16, 16) == 0   # outside the kernel's d, dv
    f = lib.la_identity_linear_fwd
    need = ws(1, 1, 8, 16, 64)
    ok = [P, P, P, 1, P, 1, 1, 1, 8, 16, 64, 0.25, P, need, None]

    def call(i, x):
        a = list(ok)
        a[i] = x
        return f(*a)

    assert call(0, None) == -1
    assert call(3, 0) == -3                              # fp32 inputs
    assert call(9, 48) == -5                             # d
    assert call(10, 16) == -5                            # dv
    assert call(11, float("inf")) == -4
    assert call(4, ctypes.c_void_p(24)) == -8            # out not 16-byte aligned
    assert call(12, None) == -6
    assert call(13, need - 1) == -6
    assert call(8, 0) == 0                               # N = 0


def test_parallel_pack_and_packed_argument_errors():
    lib = _lib()
    need = lib.la_based_parallel_workspace_bytes(1, 1, 8, 16, 64, 1)
    pack = lib.la_based_parallel_pack
    assert pack(None, P, 1, 1, 1, 8, 16, 64, P, need, None) == -1
    assert pack(P, None, 1, 1, 1, 8, 16, 64, P, need, None) == -1
    assert pack(P, P, 1, 1, 1, 8, 16, 64, None, need, None) == -6
    assert pack(ctypes.c_void_p(24), P, 1, 1, 1, 8, 16, 64, P, need, None) == -8   # k not 16-byte aligned
    assert pack(P, ctypes.c_void_p(20), 1, 1, 1, 8, 16, 64, P, need, None) == -8   # v not 8-byte aligned
    assert pack(P, P, 0, 1, 1, 8, 16, 64, None, 0, None) == 0                       # fp32: nothing to pack
    f = lib.la_based_parallel_fwd_packed
    a = [P, P, P, 1, P, 1, None, 1, 1, 8, 16, 64, 0.25, 1e-6, 1, P, need, None]
    a_bad = list(a)
    a_bad[4] = ctypes.c_void_p(40)                                               # out 8- but not 16-byte aligned
    assert f(*a_bad) == -8
    a_bad = list(a)
    a_bad[15] = None
    assert f(*a_bad) == -6


def test_parallel_workspace_sizes():
    lib = _lib()
    ws = lib.la_based_parallel_workspace_bytes
    # per (b, h) and 64-key block: fp16 V^T (dv rows padded to 68 keys, whole 1 KB units) and
    # an fp32 record of statistics (column sums of V, sums of k, the k k^T triangle, padding)
    assert ws(2, 16, 8192, 16, 64, 1) == 32 * 128 * (9216 + 4 * (64 + 160))
    assert ws(1, 1, 65, 16, 32, 1) == 2 * (5120 + 4 * (32 + 160))
    assert ws(1, 1, 64, 16, 64, 0) == 0        # fp32 inputs: no workspace
    # other bf16 shapes (register-staged kernel): 64 partial maxima of |v| per head
    assert ws(1, 1, 64, 32, 64, 1) == 256       # d != 16
    assert ws(1, 1, 64, 16, 60, 1) == 256       # dv % 8 != 0
    assert ws(2, 3, 64, 16, 72, 1) == 6 * 256   # dv > 64
    assert ws(0, 1, 64, 16, 64, 1) == 0


def test_sliding_argument_errors():
    lib = _lib()
    f = lib.la_sliding_window_fwd

    def call(q=P, W=64, scale=0.125, d=64, dv=64, N=8, dt=1):
        return f(q, P, P, dt, P, 1, 1, 1, N, d, dv, W, scale, None)

    assert call(q=None) == -1
    assert call(W=0) == -4
    assert call(scale=-1.0) == -4
    assert call(d=0) == -2
    assert call(dt=3) == -3
    assert call(d=256) == -5
    assert call(N=0) == 0


def test_chunked_argument_errors():
    lib = _lib()
    f = lib.la_based_chunked_fwd

    def call(q=P, chunk=64, d=16, dv=64, N=8, ws=P, wsb=1 << 30, scale=0.25, eps=1e-6):
        return f(q, P, P, 1, P, 1, 1, 1, N, d, dv, chunk, scale, eps, 0, ws, wsb, None, None)

    assert call(q=None) == -1
    assert call(chunk=0) == -2
    assert call(scale=0.0) == -4
    assert call(N=0) == 0


def test_chunked_chunk_argument():
    """chunk is the reference's chunk_size: any value >= 1 is accepted (the recurrence gives the
    same function for every chunk size) and the chunk the kernels run is reported."""
    lib = _lib()
    assert lib.la_based_chunked_chunk_used(0) == -2
    assert lib.la_based_chunked_chunk_used(-5) == -2
    for c in (1, 16, 64, 100, 128, 256, 4096):
        assert lib.la_based_chunked_chunk_used(c) == 128
    # the workspace does not depend on the requested chunk
    sizes = {lib.la_based_chunked_workspace_bytes(2, 16, 8192, 16, 64, c) for c in (1, 64, 128, 1000)}
    assert len(sizes) == 1
    f = lib.la_based_chunked_fwd
    assert f(P, P, P, 1, P, 1, 2, 16, 8192, 16, 64, 0, 0.25, 1e-6, 0, P, 1 << 30, None, None) == -2


def test_chunked_noalloc_argument_errors():
    """The no-allocation chunked entry point validates like la_based_chunked_fwd and rejects
    shapes whose scratch exceeds its fixed device array before touching the device."""
    lib = _lib()
    f = lib.la_based_chunked_fwd_noalloc

    def call(q=P, chunk=64, d=16, dv=64, B=2, H=16, N=8, scale=0.25, eps=1e-6, dt=1):
        return f(q, P, P, dt, P, 1, B, H, N, d, dv, chunk, scale, eps, 1, None, None)

    assert call(q=None) == -1
    assert call(chunk=0) == -2
    assert call(d=65) == -5           # above the segment-state path's 64
    assert call(dv=129) == -5
    assert call(N=0) == 0
    assert call(dt=5) == -3
    # largest scratch need below the limit: 511 heads x 2 segments of 24 KiB records
    assert lib.la_based_chunked_workspace_bytes_dt(1, 511, 256, 16, 64, 64, 1) <= (32 << 20)
    # the segment-state path (d != 16, fp32) needs scratch that grows with B*H*N: refused above
    # the fixed array, before the device is touched
    assert lib.la_based_chunked_workspace_bytes_dt(2, 16, 8192, 64, 64, 64, 1) > (32 << 20)
    assert call(d=64, dv=64, B=2, H=16, N=8192) == -10
    assert call(d=16, dv=64, B=8, H=16, N=65536, dt=0) == -10


def test_lds_copy_carries_its_wait_states():
    """The global -> LDS copies are inline assembly, in front of which the compiler inserts no
    wait states: the copy itself must hold the five that a VALU write of its descriptor SGPRs
    needs, and it must be the only LDS-DMA instruction written by hand."""
    import glob
    csrc = os.path.join(ROOT, "trainium-linear-attention_amd", "csrc")
    hits = []
    for path in sorted(glob.glob(os.path.join(csrc, "*.hip")) + glob.glob(os.path.join(csrc, "*.hpp"))):
        text = open(path).read()
        for m in re.finditer(r"asm volatile\((.*?)\);", text, re.S):
            if "lds\"" in m.group(1) or "offen lds" in m.group(1):
                hits.append((os.path.basename(path), m.group(1)))
    assert len(hits) == 1 and hits[0][0] == "la_common.hpp", hits
    nops = re.findall(r"s_nop (\d+)", hits[0][1])
    assert nops and int(nops[0]) >= 4
    assert hits[0][1].index("s_nop") < hits[0][1].index("buffer_load")


def test_reference_import_line():
    """The reference's callers import the dense function and the NKI wrapper by these names
    (benchmarks/based_attention_benchmark.py:19)."""
    from kernels.pytorch_attention import ref_based_attn, solution_nki  # noqa: F401
    import torch
    q = torch.zeros(1, 1, 4, 16)
    with pytest.raises(RuntimeError):
        ref_based_attn(q, q, q)


def test_feature_map_argument_errors():
    lib = _lib()
    f = lib.la_taylor_feature_map
    assert f(None, 0, P, 0, 4, 16, None) == -1
    assert f(P, 0, P, 0, -1, 16, None) == -2
    assert f(P, 0, P, 0, 4, 0, None) == -2
    assert f(P, 5, P, 0, 4, 16, None) == -3
    assert f(P, 0, P, 0, 4, 200, None) == -5
    assert f(P, 0, P, 0, 0, 16, None) == 0
    # rows * F beyond 2^40 elements (and far beyond, where the product would overflow int64)
    assert f(P, 0, P, 0, (1 << 40) // 153 + 1, 16, None) == -2
    assert f(P, 0, P, 0, (1 << 62), 16, None) == -2


def test_python_wrappers_refuse_cpu_tensors():
    import torch
    import kernels
    q = torch.zeros(1, 1, 4, 16)
    with pytest.raises(RuntimeError):
        kernels.solution_nki(q, q, q)
    with pytest.raises(RuntimeError):
        kernels.nki_sliding_window_attn(q, q, q)
    with pytest.raises(RuntimeError):
        kernels.chunked_nki_numerator(q, q, q)
    with pytest.raises(RuntimeError):
        kernels.taylor_feature_map(q)


def test_chunked_workspace_by_dtype():
    """The workspace query per input type: the bf16 d = 16 recurrence's, the segment-state path's
    for other head dims and for fp32 (its fp32 prefixes); the legacy query covers both types;
    one-segment sequences need none on the segment-state path."""
    lib = _lib()
    f, g = lib.la_based_chunked_workspace_bytes_dt, lib.la_based_chunked_workspace_bytes
    b16 = f(2, 16, 8192, 16, 64, 64, 1)
    f32 = f(2, 16, 8192, 16, 64, 64, 0)
    assert 0 < b16 < f32 and g(2, 16, 8192, 16, 64, 64) == max(b16, f32)
    assert f(2, 16, 512, 64, 64, 64, 1) == 0 and f(2, 16, 512, 64, 64, 64, 0) == 0   # one segment
    assert f(1, 1, 1025, 64, 128, 64, 0) > f(1, 1, 1025, 64, 128, 64, 1) > 0
    assert f(1, 1, 8192, 65, 64, 64, 1) == (1 << 64) - 1       # above the path's d
    assert f(1, 1, 8192, 16, 64, 64, 7) == (1 << 64) - 1       # unknown type
