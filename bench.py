"""Benchmark of the MI355X BASED kernels; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--configs all|none]

Headline workload: fused causal BASED forward (la_based_parallel_fwd) at B=2, H=16, N=8192,
d=16, dv=64, bf16 inputs and output, fp32 accumulation -- one "step" is one full forward
over that batch, inputs resident in HBM.  ``value`` is TFLOP/s of algorithmic work
(causal pairs x 2(d+dv) flop); ``roofline`` compares it with the bf16 dense MFMA peak.
``per_config`` adds ms/call, TFLOP/s and roofline fraction for every benchmark
configuration (fp32 parallel, bf16 parallel, chunked, sliding, long-context chunked).
``cpu_baseline`` times the CPU restatement of the reference's PyTorch path over the whole
headline workload (repeated to at least 10 s), on this host's cores.

GPU time is measured with HIP events on the stream the kernels are launched on, around K
back-to-back calls after W warm-up calls and at least --settle-ms (30) ms of back-to-back
untimed calls, so that the card's clock has settled after the step from idle to load; HBM-bound configurations rotate through several
input sets so that repeated calls do not run out of the 256 MB Infinity Cache.  Each ``per_config``
entry is the median of 5 such timed regions (``ms_reps``); the headline line times one.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "trainium-linear-attention_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3      # MI355X fp32 matrix
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E

METRIC = "BASED fwd ms + TFLOP/s at B=2,H=16,N=8192,d=16,dv=64 (% MFMA/HBM roofline)"

# (name, kind, B, H, N, d, dv, dtype, seed, chunk, window, prescale)
CONFIGS = [
    ("parallel_fp32_b1h4n1024", "parallel", 1, 4, 1024, 16, 64, "f32", 0, 64, 64, True),
    ("parallel_bf16_b2h16n2048", "parallel", 2, 16, 2048, 16, 64, "bf16", 1, 64, 64, True),
    ("chunked_bf16_b2h16n8192", "chunked", 2, 16, 8192, 16, 64, "bf16", 2, 64, 64, True),
    ("sliding_w64_bf16_b2h16n4096", "sliding", 2, 16, 4096, 64, 64, "bf16", 3, 64, 64, False),
    ("chunked_bf16_b1h16n65536", "chunked", 1, 16, 65536, 16, 64, "bf16", 4, 128, 64, True),
]
HEADLINE = ("parallel_b2h16n8192", "parallel", 2, 16, 8192, 16, 64, "bf16", 2, 64, 64, True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5,
                    help="untimed calls before each timed region (at least --settle-ms of calls run in any case)")
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="minimum milliseconds of back-to-back untimed calls before each timed region")
    ap.add_argument("--rotate", type=int, default=4, help="input sets cycled through for HBM-bound configs")
    ap.add_argument("--configs", choices=["all", "none"], default="all")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-chunk-heads", type=int, default=2,
                    help="heads per call of the CPU baseline (bounds its memory); it covers all heads")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run torch copies of MIB MiB (steps + warmup times): the known-size reference kernel "
                         "that scales FETCH_SIZE / WRITE_SIZE counters into HBM bytes")
    ap.add_argument("--only", default=None,
                    help="comma-separated configuration names (or 'headline') to measure alone, e.g. for profiling")
    ap.add_argument("--layer", action="store_true",
                    help="only time the full BASED layer (linear attention + sliding-window softmax, the sum "
                         "taken in the sliding kernel's store) against the two branches run and added apart")
    ap.add_argument("--decode", action="store_true",
                    help="only time one decode step (la_based_decode_step{,_ws}, d16 dv64) on the exported state")
    ap.add_argument("--identity", action="store_true",
                    help="only time the identity-map linear attention numerator (la_identity_linear_fwd) at "
                         "B2 H16 N8192 d16 dv64 bf16 against its HBM roofline")
    ap.add_argument("--clock-transient", action="store_true",
                    help="only time single calls of the headline attention kernel: 60 back to back from idle, then 20 "
                         "after 20 ms idle gaps (the step from idle to load that --settle-ms waits out)")
    ap.add_argument("--general", action="store_true",
                    help="time the segment-state chunked path (d != 16, fp32) beside the fused kernel")
    ap.add_argument("--crossover", action="store_true",
                    help="only sweep sequence lengths: whole parallel forward vs chunked forward (d=16, dv=64, bf16), "
                         "the measurement behind solution()'s dispatch threshold")
    return ap.parse_args()


def make_inputs(B, H, N, d, dv, dtype, seed, prescale, device):
    """Seeded N(0,1) q, k, v drawn on the CPU in the order q, k, v; BASED configurations divide
    q and k by sqrt(d) (the op then applies its own 1/sqrt(d))."""
    import torch

    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, N, d, generator=g)
    k = torch.randn(B, H, N, d, generator=g)
    v = torch.randn(B, H, N, dv, generator=g)
    if prescale:
        q = q / math.sqrt(d)
        k = k / math.sqrt(d)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    return q.to(tdt).to(device), k.to(tdt).to(device), v.to(tdt).to(device)


def feature_dim(d, symmetric=True):
    return 1 + d + (d * (d + 1) // 2 if symmetric else d * d)


def work(kind, B, H, N, d, dv, esz, chunk, window):
    """Algorithmic FLOP and HBM bytes of one call (q, k, v read once, out written once)."""
    BH = B * H
    if kind == "parallel":
        flop = BH * N * (N + 1) / 2 * 2 * (d + dv)
    elif kind == "chunked":
        flop = BH * N * (4 * feature_dim(d, symmetric=False) * dv + (chunk + 1) * (d + dv))
    else:
        W = window
        pairs = sum(min(t + 1, W) for t in range(N)) if N <= 1 << 20 else N * W
        flop = BH * pairs * 2 * (d + dv)
    nbytes = BH * N * (2 * d + 2 * dv) * esz
    return flop, nbytes


class Call:
    """One preallocated kernel launch through the C ABI."""

    def __init__(self, kind, q, k, v, chunk, window, out_f32=False, main_only=False):
        import torch

        from kernels import _lib

        self.L = _lib.lib()
        self.kind = kind
        B, H, N, d = q.shape
        dv = v.shape[-1]
        self.args_shape = (B, H, N, d, dv)
        self.q, self.k, self.v = q, k, v
        odt = torch.float32 if out_f32 else q.dtype
        self.out = torch.empty(B, H, N, dv, dtype=odt, device=q.device)
        self.dt = _lib.dtype_code(q.dtype)
        self.odt = _lib.dtype_code(odt)
        self.stream = torch.cuda.current_stream(q.device).cuda_stream
        self.chunk, self.window = chunk, window
        self.scale = 1.0 / math.sqrt(d)
        self.ws = None
        self.ws_bytes = 0
        self.main_only = main_only
        if kind == "parallel":
            nb = int(self.L.la_based_parallel_workspace_bytes(B, H, N, d, dv, self.dt))
            self.ws_bytes = nb
            self.ws = torch.empty(max(nb, 16), dtype=torch.uint8, device=q.device) if nb else None
            if main_only:
                # the attention kernel alone: K/V pre-pass done once here, outside the timed calls
                rc = self.L.la_based_parallel_pack(k.data_ptr(), v.data_ptr(), self.dt, B, H, N, d, dv,
                                                   self.ws.data_ptr() if self.ws is not None else None, self.ws_bytes,
                                                   self.stream)
                _lib.check(rc, "la_based_parallel_pack")
        if kind == "chunked":
            nb = int(self.L.la_based_chunked_workspace_bytes(B, H, N, d, dv, chunk))
            if nb == (1 << 64) - 1:
                raise RuntimeError("chunked kernel unsupported for this shape")
            self.ws_bytes = nb
            self.ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=q.device)
        self._check = _lib.check

    def __call__(self):
        B, H, N, d, dv = self.args_shape
        L = self.L
        if self.kind == "parallel":
            fn = L.la_based_parallel_fwd_packed if self.main_only else L.la_based_parallel_fwd
            rc = fn(self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.dt,
                                         self.out.data_ptr(), self.odt, None, B, H, N, d, dv, self.scale, 1e-6, 1,
                                         self.ws.data_ptr() if self.ws is not None else None, self.ws_bytes,
                                         self.stream)
        elif self.kind == "chunked":
            rc = L.la_based_chunked_fwd(self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.dt,
                                        self.out.data_ptr(), self.odt, B, H, N, d, dv, self.chunk, self.scale, 1e-6, 1,
                                        self.ws.data_ptr(), self.ws_bytes, None, self.stream)
        else:
            rc = L.la_sliding_window_fwd(self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.dt,
                                         self.out.data_ptr(), self.odt, B, H, N, d, dv, self.window, self.scale,
                                         self.stream)
        if rc != 0:
            self._check(rc, self.kind)


# Minimum duration of the warm-up before a timed region.  From idle, back-to-back calls of the
# headline attention kernel run ~180 us, slow to ~215 us between the 10th and 20th call (the
# card's clock controller reacting to the load step) and settle at ~185 us after ~10 ms; with
# idle gaps every call takes ~181 us.  Timing starts once the clock has settled.
SETTLE_MS = 30.0
# timed regions per benchmark configuration (`per_config` reports their median); the headline
# line times exactly --steps calls once
CONFIG_REPS = 5


def time_calls(calls, steps, warmup, settle_ms=None, reps=1):
    """Mean ms per call over ``steps`` back-to-back launches (HIP events on the launch stream),
    after at least ``warmup`` untimed calls and at least ``settle_ms`` of back-to-back work.  With
    ``reps`` > 1: that many timed regions of ``steps`` calls one after another, and the list of
    their means."""
    import torch

    settle_ms = SETTLE_MS if settle_ms is None else settle_ms
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    i = 0
    while i < warmup or (time.perf_counter() - t0) * 1e3 < settle_ms:
        calls[i % len(calls)]()
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()   # host time then tracks the GPU's
    torch.cuda.synchronize()
    out = []
    for _ in range(reps):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(steps):
            calls[i % len(calls)]()
        end.record()
        torch.cuda.synchronize()
        out.append(start.elapsed_time(end) / steps)
    return out[0] if reps == 1 else out


def chunk_run(chunk):
    """Tokens per chunk the chunked kernels run for a requested chunk size."""
    c = int(_lib_handle().la_based_chunked_chunk_used(int(chunk)))
    if c < 1:
        raise RuntimeError(f"invalid chunk {chunk}")
    return c


def measure(cfg, steps, warmup, rotate, device, main_only=False, reps=1):
    """ms per call of one configuration; with reps > 1 the median of that many timed regions of
    ``steps`` calls each (their means in ``ms_reps``)."""
    name, kind, B, H, N, d, dv, dt, seed, chunk, window, prescale = cfg
    esz = 2 if dt == "bf16" else 4
    crun = chunk_run(chunk) if kind == "chunked" else chunk
    # algorithmic work at the chunk size the configuration states (the recurrence computes the
    # same function at any chunk size; the chunk the kernels run is reported beside it)
    flop, nbytes = work(kind, B, H, N, d, dv, esz, chunk, window)
    hbm_bound = kind != "parallel"
    nsets = rotate if hbm_bound else 1
    calls = []
    for r in range(nsets):
        q, k, v = make_inputs(B, H, N, d, dv, dt, seed + 1000 * r, prescale, device)
        calls.append(Call(kind, q, k, v, chunk, window, main_only=main_only))
    ms_reps = time_calls(calls, steps, warmup, reps=reps) if reps > 1 else None
    ms = statistics.median(ms_reps) if reps > 1 else time_calls(calls, steps, warmup)
    peak = PEAK_BF16_TFLOPS if dt == "bf16" else PEAK_FP32_TFLOPS
    t_mfma = flop / (peak * 1e12)
    t_hbm = nbytes / (PEAK_HBM_GBS * 1e9)
    sec = ms * 1e-3
    res = {
        "ms": round(ms, 5),
        "tflops": round(flop / sec / 1e12, 3),
        "gbs": round(nbytes / sec / 1e9, 1),
        "bound": "mfma" if t_mfma >= t_hbm else "hbm",
        "roofline_frac": round(max(t_mfma, t_hbm) / sec, 4),
        "flop": flop,
        "bytes": nbytes,
        "shape": {"B": B, "H": H, "N": N, "d": d, "dv": dv, "dtype": dt,
                  **({"chunk": chunk, "chunk_run": crun} if kind == "chunked" else {}),
                  **({"window": window} if kind == "sliding" else {})},
        "input_sets": nsets,
    }
    if ms_reps is not None:
        res["ms_reps"] = [round(x, 5) for x in ms_reps]
    if kind == "chunked":
        res["tflops_f153"] = round(B * H * N * (4 * feature_dim(d) * dv + (chunk + 1) * (d + dv)) / sec / 1e12, 3)
    del calls
    torch_empty_cache()
    return res


# (B, H) pairs and sequence lengths of the crossover sweep (the reference sweeps 256 .. 16384 at B=1, H=2)
CROSSOVER_BH = [(1, 2), (2, 16), (8, 16)]
CROSSOVER_N = [256, 512, 1024, 2048, 4096, 8192, 16384]


def clock_transient(device):
    """Per-call microseconds of the headline attention kernel (V pre-pass done once): 60 calls
    back to back after 0.5 s idle, then 20 calls each after a 20 ms idle gap."""
    import torch

    name, kind, B, H, N, d, dv, dt, seed, chunk, window, prescale = HEADLINE
    q, k, v = make_inputs(B, H, N, d, dv, dt, seed, prescale, device)
    call = Call(kind, q, k, v, chunk, window, main_only=True)
    for _ in range(3):
        call()
    torch.cuda.synchronize()

    def per_call(n, gap_s):
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        for a, b in ev:
            if gap_s:
                torch.cuda.synchronize()
                time.sleep(gap_s)
            a.record()
            call()
            b.record()
        torch.cuda.synchronize()
        return [round(a.elapsed_time(b) * 1000, 1) for a, b in ev]

    time.sleep(0.5)
    b2b = per_call(60, 0.0)
    time.sleep(0.5)
    gaps = per_call(20, 0.02)
    return {"clock_transient": {"kernel": "based_parallel_bf16_kernel", "shape": "B2 H16 N8192 d16 dv64 bf16",
                                "back_to_back_us": b2b, "after_20ms_idle_us": gaps}}


def crossover(steps, warmup, rotate, device):
    """ms per call of the whole parallel forward and of the normalised chunked forward over
    CROSSOVER_N for each of CROSSOVER_BH, and per (B, H) the shortest length from which the
    chunked kernel is faster at every longer length measured."""
    rows, first = [], {}
    for B, H in CROSSOVER_BH:
        best = None
        for N in CROSSOVER_N:
            ms = {kind: measure((kind, kind, B, H, N, 16, 64, "bf16", 7, 64, 64, True), steps, warmup, rotate,
                                device)["ms"] for kind in ("parallel", "chunked")}
            rows.append({"B": B, "H": H, "N": N, "parallel_ms": ms["parallel"], "chunked_ms": ms["chunked"]})
            print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
            if ms["chunked"] < ms["parallel"]:
                best = N if best is None else best
            else:
                best = None
        first[f"B{B}H{H}"] = best
    return {"crossover": rows, "chunked_faster_from": first}


# shapes of the segment-state chunked path (head dims other than 16, fp32 inputs):
# (B, H, N, d, dv, dtype); the fused kernel is timed beside it up to N = 8192
GENERAL_SHAPES = [(2, 16, 8192, 64, 64, "bf16"), (1, 16, 65536, 64, 64, "bf16"), (2, 16, 8192, 32, 128, "bf16"),
                  (2, 16, 8192, 16, 64, "f32"), (1, 16, 65536, 16, 64, "f32")]
GENERAL_SEGMENT = 512   # tokens per segment: the span of the path's quadratic part


def general_bench(steps, warmup, device):
    """ms per call of la_based_chunked_fwd on the segment-state path and of the fused parallel
    kernel (N <= 8192) on the same inputs; TFLOP/s with the chunked FLOP count of the benchmark
    configurations, F = 1 + d + d^2 and the segment as the quadratic span."""
    rows = []
    for B, H, N, d, dv, dt in GENERAL_SHAPES:
        q, k, v = make_inputs(B, H, N, d, dv, dt, 21, True, device)
        esz = 2 if dt == "bf16" else 4
        flop, _ = work("chunked", B, H, N, d, dv, esz, GENERAL_SEGMENT, 64)
        row = {"B": B, "H": H, "N": N, "d": d, "dv": dv, "dtype": dt}
        ms = time_calls([Call("chunked", q, k, v, 64, 64)], steps, warmup)
        row["chunked_ms"] = round(ms, 5)
        row["chunked_tflops"] = round(flop / (ms * 1e-3) / 1e12, 2)
        if N <= 8192:
            pflop, _ = work("parallel", B, H, N, d, dv, esz, 64, 64)
            pms = time_calls([Call("parallel", q, k, v, 64, 64)], steps, warmup)
            row["parallel_ms"] = round(pms, 5)
            row["parallel_tflops"] = round(pflop / (pms * 1e-3) / 1e12, 2)
        rows.append(row)
        print(json.dumps(row), file=sys.stderr, flush=True)
        del q, k, v
        torch_empty_cache()
    return {"general": rows}


# full BASED layer shapes: (B, H, N, d of the linear branch, d_sw of the softmax branch, dv, window)
LAYER_SHAPES = [(2, 16, 8192, 16, 64, 64, 64), (2, 16, 2048, 16, 64, 64, 64)]


def layer_bench(steps, warmup, device):
    """ms per call of kernels.based_layer_attn and of the unfused composition (solution() and
    nki_sliding_window_attn in bf16, then a torch add), same inputs."""
    import torch

    import kernels as K

    rows = []
    for B, H, N, d, d_sw, dv, W in LAYER_SHAPES:
        q, k, v = make_inputs(B, H, N, d, dv, "bf16", 11, True, device)
        q_sw, k_sw, _ = make_inputs(B, H, N, d_sw, 1, "bf16", 12, False, device)
        fused = lambda: K.based_layer_attn(q, k, v, window_size=W, q_sw=q_sw, k_sw=k_sw)
        apart = lambda: K.solution(q, k, v) + K.nki_sliding_window_attn(q_sw, k_sw, v, window_size=W)
        row = {"B": B, "H": H, "N": N, "d": d, "d_sw": d_sw, "dv": dv, "window": W}
        for name, fn in (("layer_ms", fused), ("apart_ms", apart)):
            row[name] = round(time_calls([fn], steps, warmup), 5)
        rows.append(row)
        del q, k, v, q_sw, k_sw
        torch_empty_cache()
    return {"layer": rows}


def _lib_handle():
    from kernels import _lib

    return _lib.lib()


def decode_bench(steps, warmup, device):
    """ms per decode step (one token per head) at serving batches and at the headline's heads;
    HBM-bound: the fp32 state is read and written once, 2 x 4 F (dv + 1) bytes per head.
    `ms`: la_based_decode_step_ws, `ms_one_group`: la_based_decode_step.  A state of at most
    10240 floats per head (d16 dv64) is held in LDS by one 1024-thread work-group in both;
    larger ones (dv128) go through 256-thread work-groups, whose rows the workspace entry point
    splits over several work-groups when the batch is small,
    `ms_graph`: 16 steps of the Python wrapper captured in one HIP graph and replayed (no host
    launch cost), `ms_python_wrapper`: the wrapper called eagerly."""
    import torch

    import kernels as K

    rows = []
    for B, H, dv in [(2, 16, 64), (8, 16, 64), (64, 16, 64), (2, 16, 128), (64, 16, 128)]:
        d, F = 16, K.feature_dim(16)
        g = torch.Generator(device=device).manual_seed(3)
        q, k, v = (torch.randn(B, H, n, generator=g, device=device).bfloat16() * 0.5 for n in (d, d, dv))
        st = torch.zeros(B, H, F, dv + 1, device=device)
        out = torch.empty(B, H, dv, dtype=torch.bfloat16, device=device)
        L = _lib_handle()
        stream = torch.cuda.current_stream(device).cuda_stream
        need = int(L.la_based_decode_workspace_bytes(B, H, d, dv))
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=device)

        def abi_ws():
            rc = L.la_based_decode_step_ws(q.data_ptr(), k.data_ptr(), v.data_ptr(), 1, st.data_ptr(), out.data_ptr(),
                                           1, B, H, d, dv, 1e-6, 1, ws.data_ptr(), need, stream)
            if rc != 0:
                raise RuntimeError(f"la_based_decode_step_ws: {rc}")

        def abi_one():
            rc = L.la_based_decode_step(q.data_ptr(), k.data_ptr(), v.data_ptr(), 1, st.data_ptr(), out.data_ptr(), 1,
                                        B, H, d, dv, 1e-6, 1, stream)
            if rc != 0:
                raise RuntimeError(f"la_based_decode_step: {rc}")

        ms = time_calls([abi_ws], steps, warmup)
        ms_one = time_calls([abi_one], steps, warmup)
        ms_py = time_calls([lambda: K.based_decode_step(q, k, v, st)], steps, warmup)
        graph_steps = 16
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            K.based_decode_step(q, k, v, st)
        torch.cuda.current_stream(device).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(graph_steps):
                K.based_decode_step(q, k, v, st)
        ms_graph = time_calls([graph.replay], max(1, steps // graph_steps), 2) / graph_steps
        nbytes = 2 * B * H * F * (dv + 1) * 4
        rows.append({"B": B, "H": H, "d": d, "dv": dv, "workspace_bytes": need, "ms": round(ms, 5),
                     "ms_one_group": round(ms_one, 5), "ms_graph": round(ms_graph, 5),
                     "ms_python_wrapper": round(ms_py, 5), "state_bytes_moved": nbytes,
                     "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)})
    return {"decode": rows}


def identity_bench(steps, warmup, rotate, device):
    """ms per call of the identity-map numerator; HBM-bound: algorithmic bytes = q, k, v read and
    out written once (the per-block state records come on top)."""
    import kernels as K

    B, H, N, d, dv = 2, 16, 8192, 16, 64
    sets = [make_inputs(B, H, N, d, dv, "bf16", 21 + r, True, device) for r in range(rotate)]
    calls = [(lambda s=s: K.identity_linear_attn(*s)) for s in sets]
    ms = time_calls(calls, steps, warmup)
    nbytes = B * H * N * (2 * d + 2 * dv) * 2
    flop = B * H * N * (4 * d * dv + 65 * (d + dv))   # Q S and state update, plus the causal 64-token block
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"identity": {"shape": {"B": B, "H": H, "N": N, "d": d, "dv": dv}, "ms": round(ms, 5),
                         "gbs": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4), "bytes": nbytes,
                         "tflops": round(flop / (ms * 1e-3) / 1e12, 2), "input_sets": rotate}}


def torch_empty_cache():
    import torch

    torch.cuda.empty_cache()


def cpu_threads():
    """Threads for the CPU baseline and a description of the host CPU.  A job on a shared host
    is given its share of the cores in OMP_NUM_THREADS, while its affinity mask may show more
    cores than that share.  So: every core of the affinity mask, capped by OMP_NUM_THREADS when
    it is set."""
    aff = len(os.sched_getaffinity(0))
    threads = aff
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        threads = min(threads, int(env))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return max(1, threads), {"cpu_model": model, "affinity_cores": aff,
                             "omp_num_threads": env or None}


def cpu_baseline(chunk_heads, min_seconds=10.0):
    """The oracle's restatement of the reference PyTorch path (kernels/pytorch_attention.py:27-42,
    computed in bf16 as the reference does) over the whole headline workload -- all B*H heads,
    ``chunk_heads`` at a time to bound the t x t temporaries -- repeated until ``min_seconds`` of
    CPU time have passed, on this host's cores; reported as TFLOP/s of the same algorithmic count."""
    import torch

    from oracle import reference as ref

    threads, host = cpu_threads()
    torch.set_num_threads(threads)
    _, _, B, H, N, d, dv, dt, seed, _, _, prescale = HEADLINE
    q, k, v = make_inputs(B, H, N, d, dv, dt, seed, prescale, "cpu")
    q, k, v = (x.reshape(1, B * H, N, x.shape[-1]) for x in (q, k, v))
    passes = 0
    t0 = time.perf_counter()
    while True:
        for h0 in range(0, B * H, chunk_heads):
            sl = slice(h0, min(B * H, h0 + chunk_heads))
            ref.ref_based_attn(q[:, sl], k[:, sl], v[:, sl])
        passes += 1
        sec = time.perf_counter() - t0
        if sec >= min_seconds:
            break
    flop = B * H * N * (N + 1) / 2 * 2 * (d + dv) * passes
    return {
        "value": round(flop / sec / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"the whole workload ({B * H} heads at N={N} d={d} dv={dv}, {chunk_heads} heads at a time), "
                  f"restated reference ref_based_attn (kernels/pytorch_attention.py:27-42) in bf16 on CPU, "
                  f"{passes} passes in {sec:.1f} s ({sec / passes:.2f} s per pass)",
        "sample_seconds": round(sec, 3),
        **host,
    }


def cpu_config_baseline(cfg, budget_s=3.0):
    """CPU time of one configuration's call through the oracle's restatement of the reference's
    PyTorch path, on this host's cores: per (b, h) head, as many heads as fit in ``budget_s``
    (at least one), scaled to all B*H heads (heads are independent and equal in work).

    * parallel: ``ref_based_attn`` (kernels/pytorch_attention.py:27-42) in the configuration's dtype;
    * chunked: the dense phi-form ``ref_based_attn`` the reference's chunked benchmark times against
      (benchmarks/chunked_attention_benchmark.py:55-65, fp32 inside) up to N = 8192; above that
      (a t x t fp32 temporary of 17 GB per head) the oracle's chunk recurrence (fp32, the kernel's
      chunk), which follows kernels/nki_attention_chunked.py:65-109;
    * sliding: ``ref_sliding_window_attn`` (benchmarks/sliding_attention_benchmark.py:32-56)."""
    import torch

    from oracle import reference as ref

    name, kind, B, H, N, d, dv, dt, seed, chunk, window, prescale = cfg
    threads, host = cpu_threads()
    torch.set_num_threads(threads)
    q, k, v = make_inputs(B, H, N, d, dv, dt, seed, prescale, "cpu")
    q, k, v = (x.reshape(1, B * H, N, x.shape[-1]) for x in (q, k, v))
    if kind == "parallel":
        fn, what = ref.ref_based_attn, f"ref_based_attn (kernels/pytorch_attention.py:27-42) in {dt}"
    elif kind == "chunked" and N <= 8192:
        fn, what = ref.ref_based_attn_phi, "dense phi-form ref_based_attn (benchmarks/chunked_attention_benchmark.py:55-65)"
    elif kind == "chunked":
        crun = chunk_run(chunk)
        fn = lambda a, b_, c: ref.based_chunked(a, b_, c, chunk=crun)
        what = f"chunk recurrence (kernels/nki_attention_chunked.py:65-109), fp32, chunk {crun}"
    else:
        fn = lambda a, b_, c: ref.ref_sliding_window_attn(a, b_, c, window_size=window)
        what = f"ref_sliding_window_attn (benchmarks/sliding_attention_benchmark.py:32-56), window {window}"
    fn(q[:, :1], k[:, :1], v[:, :1])   # warm-up (allocator, thread pool)
    heads = 0
    t0 = time.perf_counter()
    while True:
        h = heads % (B * H)
        fn(q[:, h:h + 1], k[:, h:h + 1], v[:, h:h + 1])
        heads += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    sec = time.perf_counter() - t0
    ms = sec / heads * B * H * 1e3
    return {"ms": round(ms, 3), "cores": threads, "kind": "port",
            "sample": f"{what}, {heads} head evaluations of {B * H} heads in {sec:.2f} s after one warm-up head, "
                      f"scaled to all heads", **host}


def load_traffic(kernel):
    path = os.path.join(ROOT, "profiles", f"traffic_{kernel}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("bytes_per_launch")


def main():
    global SETTLE_MS
    args = parse()
    SETTLE_MS = args.settle_ms
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); how the path would shard over several "
              "GPUs is a design, not a launched path", file=sys.stderr)
        sys.exit(2)
    import torch

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)

    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": n * 4}))
        return

    if args.decode:
        print(json.dumps(decode_bench(args.steps, args.warmup, device)))
        return

    if args.identity:
        print(json.dumps(identity_bench(args.steps, args.warmup, args.rotate, device)))
        return

    if args.layer:
        print(json.dumps(layer_bench(args.steps, args.warmup, device)))
        return

    if args.crossover:
        print(json.dumps(crossover(args.steps, args.warmup, args.rotate, device)))
        return

    if args.general:
        print(json.dumps(general_bench(args.steps, args.warmup, device)))
        return

    if args.clock_transient:
        print(json.dumps(clock_transient(device)))
        return

    if args.only:
        names = set(args.only.split(","))
        res = {}
        for cfg in [HEADLINE] + CONFIGS:
            if cfg[0] in names or (cfg is HEADLINE and "headline" in names):
                res[cfg[0]] = measure(cfg, args.steps, args.warmup, args.rotate, device)
        print(json.dumps({"only": res}))
        return
    head = measure(HEADLINE, args.steps, args.warmup, args.rotate, device)
    # dominant kernel alone (attention kernel, V pre-pass done once outside the timed calls)
    main_k = measure(HEADLINE, args.steps, args.warmup, args.rotate, device, main_only=True)
    per_config = {}
    if args.configs == "all":
        for cfg in CONFIGS:
            try:
                per_config[cfg[0]] = measure(cfg, args.steps, args.warmup, args.rotate, device, reps=CONFIG_REPS)
            except RuntimeError as e:
                per_config[cfg[0]] = {"error": str(e)}
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_chunk_heads)
    if not args.no_cpu_baseline:
        for cfg in CONFIGS:
            res = per_config.get(cfg[0])
            if res is not None and "ms" in res:
                res["cpu_baseline"] = cpu_config_baseline(cfg)
                res["cpu_baseline"]["gpu_speedup"] = round(res["cpu_baseline"]["ms"] / res["ms"], 1)

    achieved = head["tflops"]
    line = {
        "metric": METRIC,
        "value": achieved,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "based_parallel_fwd causal B2 H16 N8192 d16 dv64 bf16 in/out, fp32 accumulate",
                   "global_batch": 2, "heads": 16, "seq_len": 8192, "d": 16, "dv": 64, "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "achieved": main_k["tflops"], "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(main_k["tflops"] / PEAK_BF16_TFLOPS, 4), "traffic": load_traffic("based_parallel"),
                     "kernel": "based_parallel_bf16_kernel", "kernel_ms": main_k["ms"]},
        "cpu_baseline": cpu,
        "per_config": per_config,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
