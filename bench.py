"""Benchmark of the mLSTM kernel backend on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--chunk-size 64] [--algo auto]
                    [--decode-steps 1000] [--no-cpu-baseline] [--no-decode] [--no-soft-cap] [--no-extra]
    python bench.py --summarize-pmc FETCH_DIR WRITE_DIR      (no GPU: reads rocprofv3 CSVs)
    python bench.py --summarize-trace TRACE_DIR              (no GPU: per-kernel durations of a kernel trace)

Prints ONE JSON line.  Headline (`value`): chunkwise mLSTM prefill tokens/s
at BASELINE config 2 (bf16 q/k/v/gates, float32 states, B4 NH8 S8192 DQK256
DV512, L=64, last states returned).  One step = one `mlstm_chunkwise` call
over the whole batch (B*S = 32768 tokens) with inputs resident in HBM; L2 and
the 256 MB Infinity Cache are flushed (512 MB write) before every timed call,
and each call (its gate-prep and single-pass kernels) is timed with HIP events
on the stream the kernels run on (the flush is queued without a host sync and
takes ~0.1 ms on the GPU, longer than the call's ~35 us host dispatch, so the
events bracket the kernels and not the host-side launch latency;
`prefill_ms_graph` is the same call replayed from a HIP graph, as a cross-check).  Before the timed calls the call runs back to back for
--warmup-seconds (default 1 s) after the --warmup calls, so the clocks have
settled.  `prefill_chunk_size_128` is the chunk_size=128 sweep and
`prefill_fused` the same call on the fused schedule (algo="fused").
The decode step (config 1, B16 NH8 DQK256 DV512) is reported beside it in
`decode`: 1000 chained steps over 6 rotating state sets (>256 MB, so the
state really streams from HBM), captured in a HIP graph.  `soft_cap` reports
the logit soft-cap (cap 30) over config 3's prefill logits [1, 2048, 50304]
bf16, a pure HBM stream; the same kernel serves as the known-size streaming
kernel that calibrates the rocprofv3 FETCH_SIZE / WRITE_SIZE counters.
`slstm_sequence` (config 4's sLSTM layer, one time-loop launch),
`mlstm_sequence` (the recurrent mLSTM time loop over 64 tokens of config 2's
heads) and `arbitrary_length` (the any-S wrapper on config 2 with S = 8255)
measure the remaining rows of the path; `slstm_conv1d_silu` and
`slstm_group_norm` the sLSTM layer's stages either side of its time loop at
config 4 (conv K 4 + SiLU over [8, 4096, 2048]; GroupNorm NH 4 x H 512), and
`mlstm_output_gate` the mLSTM output cell's RMSNorm x sigmoid(o) on config 2's
kernel output, `slstm_gate_proj` config 4's i/f gate projection with its
soft-cap (beside the reference's Linear + soft-cap composition on the GPU), and
`chunkwise_bwd` the chunkwise backward on config 2's shape (float32 arithmetic,
against the fp32 peak).  Each is timed with a cache flush before every call and
HIP events (calls of several launches replayed from a HIP graph, single launches
eagerly behind the flush) and reported against HBM.  `cfg3_stack` / `cfg4_stack` run
the random-init stacks end to end (prefill and graph-replayed greedy decode
tokens/s, and the decode step's lm_head with its soft-cap against hipBLASLt's
Linear then the soft-cap kernel).

HBM traffic (`roofline.traffic`) cannot be measured from inside the process:
it comes from two rocprofv3 --pmc passes over this script (FETCH_SIZE, then
WRITE_SIZE), each scaled by what the same counter reads for the soft-cap
stream of known size.  `--summarize-pmc` turns those CSVs into
profiles/hbm_traffic.json, which the timed run reports when its kernel and
workload match.

Roofline figures use algorithmic work only:
  prefill FLOP/call = B*NH*S*(4*DQK*DV + 2*L*(DQK+DV))      (1.6321e11 at L=64)
  prefill bytes/call = q,k,v,h (bf16) + gates (bf16) + last states (fp32)
  decode bytes/step  = 2|C| + 2|n| + 2|m| + |q|+|k|+|v|+|i|+|f|+|h|  (134,875,136)
Peaks: bf16 dense MFMA 2500 TFLOP/s, HBM 8000 GB/s.

The CPU baseline is the oracle (torch on the host cores, a restatement of the
reference's torch-native code) timed on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "xlstm-metal_amd"))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

PEAK_BF16_TFLOPS = 2500.0
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.json")
PREFILL_KERNEL = "chunkwise_pipe_kernel"
PREFILL_KERNEL_FUSED = "chunkwise_fused_kernel"
SOFT_CAP_KERNEL = "soft_cap_kernel"
CONV_KERNEL = "causal_conv1d_kernel"
GROUP_NORM_KERNEL = "group_norm_kernel"
RMS_GATE_KERNEL = "mh_rmsnorm_gate_kernel"
GATE_PROJ_KERNEL = "gate_proj_kernel"
GATE_ROWS_KERNEL = "gate_rows_kernel"  # the gate projection's row form (config 4's sLSTM gates)
# the lm_head's row form at the decode rows of configs 3 (1 x 4096) and 4 (8 x 2048), vocab 50304
LM_HEAD_VOCAB = 50304
LM_HEAD_CFG3_KERNEL = "lm_head_rows_kernel<xl::bf16_t, 1, 8>"
LM_HEAD_CFG4_KERNEL = "lm_head_rows_kernel<xl::bf16_t, 8, 4>"
CFG4_D_MODEL = 2048  # config 4's d_model: the sLSTM projection conv runs over all of it
CFG4_CONV_K = 4
SOFT_CAP_SHAPE = (1, 2048, 50304)  # config 3 prefill logits
SLSTM_KERNEL = "slstm_seq_kernel"
SEQ_KERNEL = "mlstm_recurrent_kernel"
SEQ_TOKENS = 64  # recurrent-sequence bench: tokens per call on config 2's heads


def prefill_flops(B, NH, S, DQK, DV, L):
    return B * NH * S * (4 * DQK * DV + 2 * L * (DQK + DV))


def prefill_bytes(B, NH, S, DQK, DV, esz=2):
    return (2 * B * NH * S * DQK * esz + 2 * B * NH * S * DV * esz + 2 * B * NH * S * esz
            + B * NH * (DQK * DV + DQK + 1) * 4)


def decode_bytes(B, NH, DQK, DV, esz=2, gsz=4):
    C, n, m = B * NH * DQK * DV * 4, B * NH * DQK * 4, B * NH * 4
    return 2 * C + 2 * n + 2 * m + 2 * B * NH * DQK * esz + 2 * B * NH * DV * esz + 2 * B * NH * gsz


def warm_clocks(fn, dev, seconds):
    """Runs fn back to back for `seconds` of wall time (after the step-count warm-up): the GPU's
    clocks take ~0.1 s of sustained load to settle, and the first calls after idle run 5-10 %
    slower than the steady state every later call sees."""
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(4):
            fn()
        torch.cuda.synchronize(dev)


class Flusher:
    """Writes a 512 MB buffer to evict L2 and the Infinity Cache (MALL)."""

    def __init__(self, device):
        self.buf = torch.empty(512 * 1024 * 1024 // 4, dtype=torch.float32, device=device)

    def __call__(self):
        self.buf.fill_(1.0)


PATTERN_WARM_CALLS = 60  # untimed (flush, call) pairs before a prefill entry's timed calls


def bench_prefill(args, dev, L=None, steps=None, algo=None):
    import xlstm_hip
    from xlstm_hip.workloads import CFG2, chunkwise_inputs
    cfg = CFG2
    L = L or args.chunk_size
    steps = steps or args.steps
    algo = algo or args.algo
    x = chunkwise_inputs(cfg, device=dev)
    flush = Flusher(dev)
    stream = torch.cuda.current_stream(dev)

    def call():
        return xlstm_hip.mlstm_chunkwise(*x, return_last_states=True, chunk_size=L, algo=algo)

    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize(dev)
    warm_clocks(call, dev, args.warmup_seconds)

    def timed(run, n):
        ts, wall = [], 0.0
        for _ in range(n):
            torch.cuda.synchronize(dev)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            w0 = time.perf_counter()
            flush()  # ~0.1 ms on the GPU: the host-side dispatch of the call runs behind it
            e0.record(stream)
            run()
            e1.record(stream)
            torch.cuda.synchronize(dev)
            wall += time.perf_counter() - w0
            ts.append(e0.elapsed_time(e1))
        return ts, wall

    # One mlstm_chunkwise call is two kernel launches (gate prep + single pass) behind a
    # torch.library dispatch of ~35 us on the host, which runs while the GPU still executes the
    # cache flush queued before the start event: the events bracket the two kernels.  The same
    # call replayed from a HIP graph is timed beside it (`ms_graph`): the replay adds tens of us of
    # its own between the events on this runtime (the kernels and their inputs are the same).
    # the timed pattern (flush, call) itself for a while first: after the inputs are allocated and
    # after a change of pattern the calls run up to ~15 % slower for some tens of calls
    timed(call, PATTERN_WARM_CALLS)
    times, t_wall = timed(call, steps)
    mode = "eager (host dispatch behind the cache flush)"
    ms_graph = None
    try:
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            call()
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            call()
        graph.replay()
        torch.cuda.synchronize(dev)
        timed(graph.replay, PATTERN_WARM_CALLS // 2)
        tg, _ = timed(graph.replay, max(3, steps // 2))
        ms_graph = statistics.mean(tg)
    except Exception:  # the graph figure is a cross-check only
        pass
    ms = statistics.mean(times)
    tokens = cfg.B * cfg.S
    fl = prefill_flops(cfg.B, cfg.NH, cfg.S, cfg.DQK, cfg.DV, L)
    by = prefill_bytes(cfg.B, cfg.NH, cfg.S, cfg.DQK, cfg.DV)
    return {
        "ms": ms, "ms_median": statistics.median(times), "ms_min": min(times), "wall_ms": 1e3 * t_wall / steps,
        "tokens": tokens, "flops": fl, "bytes": by, "L": L, "cfg": cfg, "mode": mode, "ms_graph": ms_graph,
    }


def bench_decode(args, dev):
    """cfg1 decode step through the C-ABI, 6 rotating state sets, HIP-graph replay."""
    from xlstm_hip import _lib
    from xlstm_hip.workloads import CFG1, step_inputs
    cfg = CFG1
    lib = _lib.load()
    B, NH, DQK, DV = cfg.B, cfg.NH, cfg.DQK, cfg.DV
    q, k, v, i, f, C, n, m = step_inputs(cfg, device=dev)
    nsets = 6
    Cs = [C.clone() for _ in range(nsets)]  # updated in place
    ns = [[n.clone(), torch.empty_like(n)] for _ in range(nsets)]
    ms_ = [[m.clone(), torch.empty_like(m)] for _ in range(nsets)]
    h = torch.empty(B, NH, DV, dtype=q.dtype, device=dev)
    scale = DQK ** -0.5

    def launch(s, parity, stream):
        a, b = parity, 1 - parity
        rc = lib.xl_mlstm_step_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), i.data_ptr(), f.data_ptr(),
                                   Cs[s].data_ptr(), ns[s][a].data_ptr(), ms_[s][a].data_ptr(), h.data_ptr(),
                                   Cs[s].data_ptr(), ns[s][b].data_ptr(), ms_[s][b].data_ptr(), B, NH, DQK, DV,
                                   scale, 1e-6, 1, 0, stream)
        _lib.check(rc, "decode bench")

    per_graph = 2 * nsets  # both ping-pong parities of every set
    mode = "hip_graph"
    graph = None
    try:
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for p in (0, 1):
                for s in range(nsets):
                    launch(s, p, side.cuda_stream)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            st = torch.cuda.current_stream(dev).cuda_stream
            for p in (0, 1):
                for s in range(nsets):
                    launch(s, p, st)
        run = graph.replay
    except Exception as exc:  # measurement method only; the kernel is the same
        mode = f"eager ({type(exc).__name__})"
        graph = None

        def run():
            st = torch.cuda.current_stream(dev).cuda_stream
            for p in (0, 1):
                for s in range(nsets):
                    launch(s, p, st)

    reps = max(1, args.decode_steps // per_graph)
    for _ in range(3):
        run()
    warm_clocks(run, dev, args.warmup_seconds)
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        run()
    e1.record(stream)
    torch.cuda.synchronize(dev)
    steps = reps * per_graph
    us = 1e3 * e0.elapsed_time(e1) / steps
    by = decode_bytes(B, NH, DQK, DV)
    # the ceiling of the step's own access pattern: xl_mlstm_step_copy_ceiling moves each set's
    # C (67 MB read, 67 MB written, in place like the step) with the step's grid, thread map and
    # 16-byte nontemporal loads and stores and nothing else; the same 6-set rotation, HIP graph
    def copy_launch(s_, stream_):
        _lib.check(lib.xl_mlstm_step_copy_ceiling(Cs[s_].data_ptr(), Cs[s_].data_ptr(), B, NH, DQK, DV, stream_),
                   "decode copy ceiling")

    copy_graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for s in range(nsets):
            copy_launch(s, side.cuda_stream)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    with torch.cuda.graph(copy_graph):
        st = torch.cuda.current_stream(dev).cuda_stream
        for s in range(nsets):
            copy_launch(s, st)
    for _ in range(3):
        copy_graph.replay()
    warm_clocks(copy_graph.replay, dev, min(0.3, args.warmup_seconds))
    torch.cuda.synchronize(dev)
    creps = max(1, args.decode_steps // nsets)
    e0.record(stream)
    for _ in range(creps):
        copy_graph.replay()
    e1.record(stream)
    torch.cuda.synchronize(dev)
    copy_us = 1e3 * e0.elapsed_time(e1) / (creps * nsets)
    return {"us_per_step": us, "steps": steps, "bytes": by, "mode": mode, "state_sets": nsets, "cfg": cfg,
            "copy_us": copy_us, "copy_bytes": 2 * Cs[0].numel() * Cs[0].element_size()}


def bench_soft_cap(args, dev):
    """Logit soft-cap (cap 30) over config 3's prefill logits, bf16, through the C-ABI."""
    from xlstm_hip import _lib
    lib = _lib.load()
    g = torch.Generator(device=dev).manual_seed(3)
    x = (40 * torch.randn(SOFT_CAP_SHAPE, generator=g, device=dev)).to(torch.bfloat16)
    y = torch.empty_like(x)
    flush = Flusher(dev)
    stream = torch.cuda.current_stream(dev)

    def call():
        _lib.check(lib.xl_soft_cap_fwd(x.data_ptr(), y.data_ptr(), x.numel(), 30.0, 1, stream.cuda_stream), "soft_cap")

    for _ in range(3):
        call()
    times = []
    for _ in range(max(5, args.steps)):
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        flush()
        e0.record(stream)
        call()
        e1.record(stream)
        torch.cuda.synchronize(dev)
        times.append(e0.elapsed_time(e1))
    us = 1e3 * statistics.mean(times)
    by = 2 * x.numel() * x.element_size()
    return {"workload": "cfg3 logit soft_cap (cap 30) [1,2048,50304] bf16", "us_per_call": us,
            "roofline": {"bound": "hbm", "achieved": by / (us * 1e-6) / 1e9, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": by / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, "bytes_per_call": by,
                         "traffic": load_traffic(SOFT_CAP_KERNEL, "cfg3 logit soft_cap (cap 30) [1,2048,50304] bf16")}}


def _timed(call, dev, steps, warmup=10, graph=True):
    """Mean / median / min HIP-event ms of `call` over `steps` runs, each after a cache flush.
    graph=True: the call is replayed from a HIP graph when it can be captured (host dispatch of
    several launches stays out of the timed region), else run eagerly.  graph=False (calls of one
    kernel launch, at most followed by a small cast): the call runs eagerly; its host-side dispatch overlaps the ~0.1 ms
    flush queued before it, and the events then bracket the kernel alone (a graph replay adds
    ~12 us of its own between the events on this runtime, measured against rocprofv3's kernel
    durations)."""
    flush = Flusher(dev)
    stream = torch.cuda.current_stream(dev)
    for _ in range(warmup):
        call()
    torch.cuda.synchronize(dev)
    mode = "hip_graph" if graph else "eager"
    try:
        if not graph:
            raise _Eager()
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            call()
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            call()
        graph.replay()
        torch.cuda.synchronize(dev)
        run = graph.replay
    except _Eager:
        run = call
    except Exception as exc:  # measurement method only; the kernels are the same
        mode, run = f"eager ({type(exc).__name__})", call
    for _ in range(warmup):  # the timed pattern itself (flush, call), untimed
        flush()
        run()
    times = []
    for _ in range(steps):
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        flush()
        e0.record(stream)
        run()
        e1.record(stream)
        torch.cuda.synchronize(dev)
        times.append(e0.elapsed_time(e1))
    return {"ms": statistics.mean(times), "ms_median": statistics.median(times), "ms_min": min(times), "mode": mode}


class _Eager(Exception):
    """Selects eager timing in _timed."""


def _hbm(by, ms):
    gbs = by / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
            "bytes_per_call": by}


def slstm_bytes():
    """cfg4 sLSTM layer: z and h (bf16) + the three gates (bf16) + last c, n, m (float32)."""
    from xlstm_hip.workloads import CFG4_SLSTM as c
    return 2 * c.B * c.S * c.NH * c.H * 2 + 3 * c.B * c.S * c.NH * 2 + c.B * c.NH * (2 * c.H + 1) * 4


def mlstm_sequence_bytes():
    """Recurrent sequence on cfg2's heads: C, n, m read and written once + q, k, v, h, gates of the tokens."""
    from xlstm_hip.workloads import CFG2 as c
    BH = c.B * c.NH
    return 2 * BH * (c.DQK * c.DV + c.DQK + 1) * 4 + BH * SEQ_TOKENS * (2 * c.DQK + 2 * c.DV + 2) * 2


def _workloads():
    from xlstm_hip.workloads import CFG2, CFG4_SLSTM as c
    return (f"cfg4 sLSTM layer sequence B{c.B} S{c.S} NH{c.NH} H{c.H} bf16",
            f"mlstm recurrent sequence, cfg2 heads B{CFG2.B} NH{CFG2.NH} DQK{CFG2.DQK} DV{CFG2.DV}, S={SEQ_TOKENS}")


def bench_slstm_sequence(args, dev):
    """sLSTM time loop over config 4's sLSTM layer (B8 S4096 NH4 H512, bf16 z / gates / h,
    float32 states from zero, last states returned): one xl_slstm_seq_fwd launch.
    Bytes: z and h (bf16) + the three gates (bf16) + last c, n, m (float32)."""
    import xlstm_hip
    from xlstm_hip.workloads import CFG4_SLSTM as c, slstm_inputs
    z, i, f, o = slstm_inputs(c, device=dev)
    t = _timed(lambda: xlstm_hip.slstm_sequence(z, i, f, o), dev, max(5, args.steps), graph=False)
    wl = _workloads()[0]
    return {"workload": wl, "us_per_call": 1e3 * t["ms"], "us_min": 1e3 * t["ms_min"],
            "tokens_per_s": c.B * c.S / (t["ms"] * 1e-3), "mode": t["mode"],
            "roofline": dict(_hbm(slstm_bytes(), t["ms"]), traffic=load_traffic(SLSTM_KERNEL, wl))}


SLSTM_STEPS = 32  # chained sLSTM steps per timed call


def bench_slstm_step(args, dev):
    """sLSTM decode step at config 4's sLSTM shape (B8 NH4 H512: bf16 z and gates, float32 c, n, m
    carried from step to step): SLSTM_STEPS chained xl_slstm_step_fwd launches per timed call (one
    HIP-graph replay).  Bytes per step: z (bf16) + three gates (bf16) + c, n, m in and out and h
    (float32, the states' dtype).  A step moves ~0.3 MB, so it is launch-latency bound."""
    import xlstm_hip
    from xlstm_hip.workloads import CFG4_SLSTM as c
    g = torch.Generator("cpu").manual_seed(c.seed)
    z = torch.randn(SLSTM_STEPS, c.B, c.NH, c.H, generator=g).to(c.dtype).to(dev)
    gates = [(torch.randn(SLSTM_STEPS, c.B, c.NH, generator=g) + off).to(c.dtype).to(dev) for off in (0.0, 3.0, 0.0)]
    st0 = (torch.zeros(c.B, c.NH, c.H, device=dev), torch.zeros(c.B, c.NH, c.H, device=dev),
           torch.zeros(c.B, c.NH, device=dev))

    def call():
        cs, ns, ms = st0
        for t in range(SLSTM_STEPS):
            _, cs, ns, ms = xlstm_hip.slstm_step(z[t], gates[0][t], gates[1][t], gates[2][t], cs, ns, ms)

    t = _timed(call, dev, max(5, args.steps))
    el = c.B * c.NH * c.H
    by = el * 2 + 3 * c.B * c.NH * 2 + 2 * (2 * el + c.B * c.NH) * 4 + el * 4
    us = 1e3 * t["ms"] / SLSTM_STEPS
    return {"workload": f"cfg4 sLSTM decode step B{c.B} NH{c.NH} H{c.H} (bf16 z/gates, fp32 states), "
                        f"{SLSTM_STEPS} chained steps per call", "us_per_step": us, "mode": t["mode"],
            "roofline": _hbm(by, us * 1e-3)}


def _cfg4_layer_stage_inputs(dev):
    from xlstm_hip.workloads import CFG4_SLSTM as c
    g = torch.Generator(device=dev).manual_seed(c.seed)
    D = CFG4_D_MODEL
    x = torch.randn(c.B, c.S, D, generator=g, device=dev).to(c.dtype)
    w = (0.5 * torch.randn(D, 1, CFG4_CONV_K, generator=g, device=dev)).to(c.dtype)
    b = torch.randn(D, generator=g, device=dev).to(c.dtype)
    return c, x, w, b


def layer_stage_work():
    """(workload, algorithmic bytes) of the layer-stage and projection launches: cfg4's conv + SiLU,
    GroupNorm and gate projection, cfg2's norm x sigmoid(o), the decode lm_heads of cfg3 / cfg4."""
    from xlstm_hip.workloads import CFG4_SLSTM as c
    D, NHH = CFG4_D_MODEL, c.NH * c.H
    conv = (f"cfg4 sLSTM conv1d K{CFG4_CONV_K} + SiLU [B{c.B}, S{c.S}, {D}] bf16",
            2 * c.B * c.S * D * 2 + D * (CFG4_CONV_K + 1) * 2)
    gn = (f"cfg4 sLSTM GroupNorm NH{c.NH} x H{c.H} over [{c.B * c.S}, {NHH}] bf16", 2 * c.B * c.S * NHH * 2 + 2 * NHH * 2)
    from xlstm_hip.workloads import CFG2 as c2
    nel = c2.B * c2.NH * c2.S * c2.DV
    rms = (f"cfg2 mLSTM output norm x sigmoid(o) [B{c2.B}, NH{c2.NH}, S{c2.S}, DH{c2.DV}] bf16",
           3 * nel * 2 + c2.NH * c2.DV * 2)
    gp = (f"cfg4 sLSTM i/f gate projection + soft-cap 15 [{c.B * c.S}, {D}] x [{2 * c.NH}, {D}] bf16",
          c.B * c.S * D * 2 + 2 * c.NH * D * 2 + c.B * c.S * 2 * c.NH * 2)
    def lm(M, Dm):  # weights, token rows, logits
        return (f"lm_head + soft-cap 30: {M} row(s) x D {Dm} x vocab {LM_HEAD_VOCAB} bf16",
                LM_HEAD_VOCAB * Dm * 2 + M * Dm * 2 + M * LM_HEAD_VOCAB * 2)
    return {CONV_KERNEL: conv, GROUP_NORM_KERNEL: gn, RMS_GATE_KERNEL: rms, GATE_PROJ_KERNEL: gp, GATE_ROWS_KERNEL: gp,
            LM_HEAD_CFG3_KERNEL: lm(1, 4096), LM_HEAD_CFG4_KERNEL: lm(8, CFG4_D_MODEL)}


def bench_slstm_conv(args, dev):
    """Config 4's sLSTM projection conv: depthwise causal conv1d (K 4) + SiLU over x [B8, S4096,
    d_model 2048] bf16, channels last (xl_causal_conv1d_fwd).  Bytes: x read and y written once,
    plus the taps and bias."""
    import xlstm_hip
    c, x, w, b = _cfg4_layer_stage_inputs(dev)
    t = _timed(lambda: xlstm_hip.causal_conv1d(x, w, b, activation="silu"), dev, max(5, args.steps), graph=False)
    wl, by = layer_stage_work()[CONV_KERNEL]
    return {"workload": wl, "us_per_call": 1e3 * t["ms"], "us_min": 1e3 * t["ms_min"], "mode": t["mode"],
            "roofline": dict(_hbm(by, t["ms"]), traffic=load_traffic(CONV_KERNEL, wl))}


def bench_group_norm(args, dev):
    """Config 4's sLSTM output GroupNorm: one group per head (NH 4 x H 512) over the kernel output
    viewed as [B8 * S4096, 2048] bf16, affine (xl_group_norm_fwd).  Bytes: h read and y written
    once, plus weight and bias."""
    import xlstm_hip
    c, x, w, b = _cfg4_layer_stage_inputs(dev)
    h = x.view(c.B * c.S, c.NH * c.H)
    gw, gb = w.reshape(-1)[: c.NH * c.H].contiguous(), b.clone()
    t = _timed(lambda: xlstm_hip.group_norm(h, c.NH, gw, gb, 1e-6), dev, max(5, args.steps), graph=False)
    wl, by = layer_stage_work()[GROUP_NORM_KERNEL]
    return {"workload": wl, "us_per_call": 1e3 * t["ms"], "us_min": 1e3 * t["ms_min"], "mode": t["mode"],
            "roofline": dict(_hbm(by, t["ms"]), traffic=load_traffic(GROUP_NORM_KERNEL, wl))}


def bench_mlstm_output_gate(args, dev):
    """The mLSTM output cell's stage after the chunkwise kernel on config 2's output: per-head
    RMSNorm of h [B4, NH8, S8192, DH512] (read in the kernel's layout), the weight and sigmoid of
    the gate pre-activation [B4, S8192, 4096], written as [B4, S8192, 4096] bf16
    (xl_mh_rmsnorm_gate_fwd).  Bytes: h and o read once, y written once, plus the weight."""
    import xlstm_hip
    from xlstm_hip.workloads import CFG2 as c
    g = torch.Generator(device=dev).manual_seed(c.seed)
    h = torch.randn(c.B, c.NH, c.S, c.DV, generator=g, device=dev).to(c.dtype)
    w = torch.randn(c.NH * c.DV, generator=g, device=dev).to(c.dtype)
    o = torch.randn(c.B, c.S, c.NH * c.DV, generator=g, device=dev).to(c.dtype)
    t = _timed(lambda: xlstm_hip.mh_rmsnorm_gate(h, w, o, 1e-6), dev, max(5, args.steps), graph=False)
    wl, by = layer_stage_work()[RMS_GATE_KERNEL]
    return {"workload": wl, "us_per_call": 1e3 * t["ms"], "us_min": 1e3 * t["ms_min"], "mode": t["mode"],
            "roofline": dict(_hbm(by, t["ms"]), traffic=load_traffic(RMS_GATE_KERNEL, wl))}


def bench_gate_proj(args, dev):
    """Config 4's sLSTM i and f gates: x_conv [B8 * S4096, 2048] bf16 times the stacked gate weights
    [8, 2048] plus bias, soft-capped at 15 (xl_gate_proj_softcap_fwd).  Bytes: x read once, the
    weights, the [32768, 8] output.  The reference's composition on the same GPU (two nn.Linear
    calls and two soft-caps, torch + hipBLASLt) is timed beside it."""
    import torch.nn.functional as F
    import xlstm_hip
    c, x, _, _ = _cfg4_layer_stage_inputs(dev)
    x2 = x.view(c.B * c.S, CFG4_D_MODEL)
    g = torch.Generator(device=dev).manual_seed(c.seed + 1)
    w = (0.05 * torch.randn(2 * c.NH, CFG4_D_MODEL, generator=g, device=dev)).to(c.dtype)
    b = torch.randn(2 * c.NH, generator=g, device=dev).to(c.dtype)
    t = _timed(lambda: xlstm_hip.gate_proj_softcap(x2, w, b, 15.0), dev, max(5, args.steps), graph=False)
    wi, wf, bi, bf = w[:c.NH], w[c.NH:], b[:c.NH], b[c.NH:]
    tr = _timed(lambda: (xlstm_hip.soft_cap(F.linear(x2, wi, bi), 15.0), xlstm_hip.soft_cap(F.linear(x2, wf, bf), 15.0)),
                dev, max(5, args.steps))
    wl, by = layer_stage_work()[GATE_PROJ_KERNEL]
    return {"workload": wl, "us_per_call": 1e3 * t["ms"], "us_min": 1e3 * t["ms_min"], "mode": t["mode"],
            "reference_composition_us": 1e3 * tr["ms"],
            "roofline": dict(_hbm(by, t["ms"]), traffic=load_traffic(GATE_PROJ_KERNEL, wl))}


def bench_mlstm_sequence(args, dev):
    """Recurrent mLSTM time loop (xl_mlstm_sequence_fwd) over 64 tokens of config 2's heads
    (B4 NH8 DQK256 DV512, bf16 q/k/v/gates) from config-1-style float32 initial states, last
    states returned.  Bytes: C, n, m read and written once + q, k, v, h, gates of the 64 tokens."""
    import xlstm_hip
    from xlstm_hip.workloads import CFG2, chunkwise_inputs
    cfg, S = CFG2, SEQ_TOKENS
    q, k, v, i, f = chunkwise_inputs(cfg, device=dev, S=S)
    g = torch.Generator("cpu").manual_seed(5)
    C = (0.1 * torch.randn(cfg.B, cfg.NH, cfg.DQK, cfg.DV, generator=g)).to(dev)
    n = torch.randn(cfg.B, cfg.NH, cfg.DQK, generator=g).abs().to(dev)
    m = torch.randn(cfg.B, cfg.NH, 1, generator=g).to(dev)
    t = _timed(lambda: xlstm_hip.mlstm_recurrent_sequence__native_fw(q, k, v, i, f, C, n, m, return_last_states=True),
               dev, max(5, args.steps), graph=False)
    wl = _workloads()[1]
    return {"workload": wl, "us_per_call": 1e3 * t["ms"], "us_min": 1e3 * t["ms_min"], "us_per_token": 1e3 * t["ms"] / S,
            "mode": t["mode"],
            "roofline": dict(_hbm(mlstm_sequence_bytes(), t["ms"]), traffic=load_traffic(SEQ_KERNEL, wl))}


def bench_cfg3_heads(args, dev):
    """The chunkwise call of one config 3 mLSTM layer (B1 NH8 S2048 DQK256 DV512, bf16, config 0's value
    distributions, last states): 8 heads x 8 column tiles are 64 workgroups for 256 CUs, so the fused
    kernel splits the sequence into 4 segments (a states-only pass over the first three, the segment
    combine, then all four from their start states).  Beside it the same call unsplit (the
    no-allocation entry point, which never splits)."""
    import xlstm_hip
    from xlstm_hip import _lib
    from xlstm_hip.workloads import CFG2, chunkwise_inputs
    B, NH, S, DQK, DV = 1, 8, 2048, CFG2.DQK, CFG2.DV
    q, k, v, i, f = chunkwise_inputs(CFG2, device=dev, S=S, B=B)
    lib = _lib.load()
    h = torch.empty(B, NH, S, DV, dtype=q.dtype, device=dev)
    cl = torch.empty(B, NH, DQK, DV, device=dev)
    nl = torch.empty(B, NH, DQK, device=dev)
    ml = torch.empty(B, NH, device=dev)

    def unsplit():
        _lib.check(lib.xl_mlstm_chunkwise_fwd_noalloc(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), i.data_ptr(), f.data_ptr(), None, None, None, h.data_ptr(),
            cl.data_ptr(), nl.data_ptr(), ml.data_ptr(), B, NH, S, DQK, DV, 64, DQK ** -0.5, 1e-6, 1, 1,
            torch.cuda.current_stream(dev).cuda_stream), "noalloc")

    t = _timed(lambda: xlstm_hip.mlstm_chunkwise(q, k, v, i, f, return_last_states=True), dev, max(10, args.steps))
    tu = _timed(unsplit, dev, max(10, args.steps))
    fl = prefill_flops(B, NH, S, DQK, DV, 64)
    return {"workload": f"cfg3 mLSTM layer chunkwise B{B} NH{NH} S{S} DQK{DQK} DV{DV} bf16",
            "us_per_call": 1e3 * t["ms"], "us_min": 1e3 * t["ms_min"], "mode": t["mode"],
            "tokens_per_s": B * S / (t["ms"] * 1e-3), "tflops": fl / (t["ms"] * 1e-3) / 1e12,
            "unsplit_us_per_call": 1e3 * tu["ms"], "split_speedup": tu["ms"] / t["ms"]}


def bwd_flops(B, NH, S, DQK, DV, L):
    """FLOP of the reference's custom backward as xl_mlstm_chunkwise_bwd runs it, per chunk: the
    recomputed states (L DQK DV), the dC recurrence (L DQK DV), the inter-chunk dV, dK, dQ products
    (3 L DQK DV), the intra-chunk Q K^T twice, dS Q and dS^T K (4 L^2 DQK) and dH~ V^T, Sbar^T dH~
    (2 L^2 DV); 2 FLOP per multiply-add."""
    NC = S // L
    return 2.0 * B * NH * NC * (5 * L * DQK * DV + 4 * L * L * DQK + 2 * L * L * DV)


FUSED_PATH = ["states scan", "stats", "dC scan", "dV, dQ, dK", "gate gradients"]


def bwd_bytes(B, NH, S, DQK, DV, L, esz=2):
    """HBM bytes of this design's backward on the path config 2 takes (bf16, 64-token chunks, DV 256
    or 512): the algorithmic bytes of its five launches (bwd_kernel_bytes), with the per-chunk
    states C and dC materialised once each (bw.py: matC_states recomputed, matDeltaC_states) in
    the 24-bit packed form, written by the scans and read once by the fused dV / dQ / dK pass."""
    kb = bwd_kernel_bytes(B, NH, S, DQK, DV, L, esz, st_esz=3)
    return sum(kb[k] for k in FUSED_PATH)


def bwd_io_bytes(B, NH, S, DQK, DV, esz=2):
    """Compulsory HBM bytes of the chunkwise backward whatever its design: q, k, v, dH and the gates
    read once, dq, dk, dv and the gate gradients written once, the last-state gradient dC_last read
    once (float32)."""
    return B * NH * S * ((2 * DQK + 2 * DV) + (2 * DQK + DV) + 4) * esz + B * NH * DQK * DV * 4


BWD_KERNELS = {  # kernel-name key -> short name, for the trace / counter summaries of the backward
    "bw_scan_bf16_kernel<xl::bf16_t, 64, 2, false, true>": "states scan",
    "bw_stats_bf16_kernel": "stats",
    "bw_scan_bf16_kernel<xl::bf16_t, 64, 2, true, true>": "dC scan",
    "bw_dv_bf16_kernel": "dV",
    "bw_dqk_bf16_kernel": "dQ, dK",
    "bw_dvqk_bf16_kernel": "dV, dQ, dK",
    "bw_gates_kernel": "gate gradients",
}


def bwd_kernel_bytes(B, NH, S, DQK, DV, L, esz=2, st_esz=4):
    """Algorithmic HBM bytes of each backward launch (bf16 q/k/v/dH/gates): what it must read and
    write once, with the per-chunk states at st_esz bytes per value (4: float32, the two-pass
    launches; 3: the 24-bit packed states of the fused path) and the partials in float32."""
    NC, BNH, ndt, nvt = S // L, B * NH, -(-DQK // 64), -(-DV // 64)
    st = NC * DQK * DV * st_esz
    g = 2 * S * esz  # i, f
    return {
        "states scan": BNH * (S * (DQK + DV) * esz + g + st + NC * (DQK + 1) * 4 + (DQK * DV + DQK + 1) * 4),
        "stats": BNH * (2 * S * DQK * esz + g + NC * (DQK + 1) * 4 + 2 * S * 4),
        "dC scan": BNH * (S * (DQK + DV) * esz + g + 2 * S * 4 + NC * 4 + DQK * DV * 4 + st + DQK * DV * st_esz),
        "dV": BNH * (2 * S * DQK * esz + 2 * S * DV * esz + st + g + 2 * S * 4 + S * DV * esz + S * nvt * 4),
        "dQ, dK": BNH * (2 * S * DQK * esz + 2 * S * DV * esz + 2 * st + g + 2 * S * 4 + 2 * S * DQK * esz
                         + S * ndt * 4),
        # the fused pass: C and dC once, q k v dH in, dq dk dv out, the dF and dI partials
        "dV, dQ, dK": BNH * (2 * S * DQK * esz + 2 * S * DV * esz + 2 * st + g + 2 * S * 4
                             + (2 * S * DQK + S * DV) * esz + S * (ndt + nvt) * 4),
        "gate gradients": BNH * (S * (ndt + nvt) * 4 + S * esz + 2 * S * esz),
    }


def bench_chunkwise_bwd(args, dev):
    """The chunkwise backward (xl_mlstm_chunkwise_bwd, the reference's custom backward) on config 2's
    shape: B4 NH8 S8192 DQK256 DV512 bf16, last-state gradient included.  Products on bf16 MFMA
    (float32 operands as bf16 hi / lo pairs), float32 accumulation; bound by the float32 state
    traffic, so the roofline is HBM bytes, with the bf16 MFMA fraction beside it."""
    from xlstm_hip.ops import mlstm_chunkwise_bwd_op
    from xlstm_hip.workloads import CFG2, chunkwise_inputs
    cfg = CFG2
    q, k, v, i, f = chunkwise_inputs(cfg, device=dev)
    g = torch.Generator("cpu").manual_seed(12)
    dh = torch.randn(cfg.B, cfg.NH, cfg.S, cfg.DV, generator=g).to(cfg.dtype).to(dev)
    dcl = torch.randn(cfg.B, cfg.NH, cfg.DQK, cfg.DV, generator=g).to(dev)

    def call():
        return mlstm_chunkwise_bwd_op(q, k, v, i, f, None, None, None, dh, dcl, cfg.DQK ** -0.5, 64, 1e-6)

    t = _timed(call, dev, max(3, args.steps // 4), warmup=2)
    fl = bwd_flops(cfg.B, cfg.NH, cfg.S, cfg.DQK, cfg.DV, 64)
    by = bwd_bytes(cfg.B, cfg.NH, cfg.S, cfg.DQK, cfg.DV, 64)
    io = bwd_io_bytes(cfg.B, cfg.NH, cfg.S, cfg.DQK, cfg.DV)
    tf = fl / (t["ms"] * 1e-3) / 1e12
    gbs = by / (t["ms"] * 1e-3) / 1e9
    gio = io / (t["ms"] * 1e-3) / 1e9
    return {"workload": f"cfg2 chunkwise backward B{cfg.B} NH{cfg.NH} S{cfg.S} DQK{cfg.DQK} DV{cfg.DV} bf16 in, "
                        "bf16 MFMA (float32 operands as hi / lo pairs), float32 accumulation",
            "ms_per_call": t["ms"], "ms_min": t["ms_min"], "mode": t["mode"],
            "tokens_per_s": cfg.B * cfg.S / (t["ms"] * 1e-3), "flops_per_call": fl,
            # against what any backward must move (inputs, gradients) and the algorithmic flop
            "roofline": {"bound": "hbm", "achieved": gio, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gio / PEAK_HBM_GBS, "bytes_per_call": io,
                         "what": "compulsory I/O: q k v dH gates dC_last in, dq dk dv di df out"},
            "mfma_bf16": {"achieved_tflops": tf, "peak": PEAK_BF16_TFLOPS, "frac": tf / PEAK_BF16_TFLOPS,
                          "what": "algorithmic flop of the custom backward (bwd_flops)"},
            # against this design's own traffic (the float32 per-chunk C and dC it materialises)
            "design_traffic": {"bytes_per_call": by, "achieved": gbs, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS}}


def bench_arbitrary_length(args, dev):
    """Any-S inference wrapper (wrap_chunkwise__arbitrary_sequence_length) on config 2 with
    S = 8192 + 63, the reference's worst tail (its split: chunk sizes 64, 32, 16 and a 15-token
    recurrent tail).  With bf16 inputs this library runs it as one fused call with a ragged last
    chunk.  Compared with the S = 8192 headline call."""
    from xlstm_hip import backend
    from xlstm_hip.workloads import CFG2, chunkwise_inputs
    cfg, S = CFG2, 8192 + 63
    q, k, v, i, f = chunkwise_inputs(cfg, device=dev, S=S)

    def call():
        return backend.wrap_chunkwise__arbitrary_sequence_length(
            backend.get_mlstm_kernel("chunkwise--native_autograd"),
            backend.get_mlstm_sequence_kernel("native_sequence__native"), backend.get_mlstm_step_kernel("native"),
            q=q, k=k, v=v, f=f, i=i, return_last_states=True, chunk_size=64)

    t = _timed(call, dev, max(5, args.steps // 2))
    fl = prefill_flops(cfg.B, cfg.NH, S, cfg.DQK, cfg.DV, 64)
    by = prefill_bytes(cfg.B, cfg.NH, S, cfg.DQK, cfg.DV)
    return {"workload": f"cfg2 any-S inference wrapper, S={S} (bf16: one fused call, ragged last 64-token chunk)",
            "ms_per_call": t["ms"], "ms_min": t["ms_min"], "tokens_per_s": cfg.B * S / (t["ms"] * 1e-3),
            "mode": t["mode"], "tflops_64_token_algorithm": fl / (t["ms"] * 1e-3) / 1e12,
            "roofline_hbm": _hbm(by, t["ms"])}


def bench_stack(args, dev, which):
    """BASELINE config 3 or 4 end to end on the random-init stack (xlstm_hip.stack): prefill tokens/s
    of the whole prompt (B x S tokens through every block, the final norm, the lm_head and the logit
    soft-cap of the last position) and greedy-decode tokens/s (one HIP-graph replay per token: every
    block's step kernels, the lm_head, the soft-cap and the argmax), both timed with HIP events."""
    from xlstm_hip.stack import CFG3_STACK, CFG4_STACK, DecodeGraph, xLSTMStack
    cfg, B, S, steps = (CFG3_STACK, 1, 2048, 256) if which == "cfg3" else (CFG4_STACK, 8, 4096, 128)
    model = xLSTMStack.random(cfg, dev, seed=3 if which == "cfg3" else 4)
    g = torch.Generator(device=dev).manual_seed(11)
    prompt = torch.randint(0, cfg.vocab, (B, S), generator=g, device=dev)
    stream = torch.cuda.current_stream(dev)
    for _ in range(2):
        logits, states = model.prefill(prompt)
    torch.cuda.synchronize(dev)
    times = []
    for _ in range(max(3, args.steps // 4)):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        logits, states = model.prefill(prompt)
        e1.record(stream)
        torch.cuda.synchronize(dev)
        times.append(e0.elapsed_time(e1))
    pre_ms = statistics.median(times)
    dg = DecodeGraph(model, states, logits.argmax(-1))
    for _ in range(4):
        dg.step()
    torch.cuda.synchronize(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        dg.graph.replay()
        dg.token.copy_(dg.next_token)
    e1.record(stream)
    torch.cuda.synchronize(dev)
    dec_ms = e0.elapsed_time(e1) / steps
    # the decode step's logit projection: the fused lm_head + soft-cap kernel against torch's Linear
    # (hipBLASLt) then the soft_cap kernel, on the same normalised rows; three copies of the weights
    # used in turn (more than the 256 MB last-level cache holds), as in decoding, where every other
    # weight of the model streams between two lm_head calls; each variant replayed from a HIP graph
    from xlstm_hip.soft_cap import lm_head_softcap, soft_cap
    xn = model.out_norm(torch.randn(B, 1, cfg.d_model, generator=g, device=dev).to(cfg.dtype))
    W0 = model.lm_head.weight
    Ws = [W0, W0.clone(), W0.clone()]
    variants = {True: lambda w: lm_head_softcap(xn, w, cfg.logit_soft_cap),
                False: lambda w: soft_cap(torch.nn.functional.linear(xn, w), cfg.logit_soft_cap)}
    lm_us = {}
    for fused, fn in variants.items():
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for w in Ws:
                fn(w)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        lg = torch.cuda.CUDAGraph()
        with torch.cuda.graph(lg):
            for w in Ws:
                fn(w)
        for _ in range(3):
            lg.replay()
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(20):
            lg.replay()
        e1.record(stream)
        torch.cuda.synchronize(dev)
        lm_us[fused] = e0.elapsed_time(e1) * 1e3 / (20 * len(Ws))
    del Ws, variants
    w_bytes = W0.numel() * W0.element_size()
    nparams = sum(p.numel() for p in model.parameters())
    n_sl = sum(cfg.is_slstm(b) for b in range(cfg.num_blocks))
    del model, states, dg
    torch.cuda.empty_cache()
    return {"workload": f"{which} random-init stack: {cfg.num_blocks} blocks ({cfg.num_blocks - n_sl} mLSTM, {n_sl} "
                        f"sLSTM), d {cfg.d_model}, vocab {cfg.vocab}, {nparams / 1e9:.2f}B params, bf16; B{B}, "
                        f"prefill {S} tokens, then {steps} greedy decode steps",
            "prefill_ms": pre_ms, "prefill_tokens_per_s": B * S / (pre_ms * 1e-3),
            "decode_ms_per_step": dec_ms, "decode_tokens_per_s": B / (dec_ms * 1e-3), "decode_steps": steps,
            "decode_mode": "hip_graph (one replay per token)",
            "lm_head_decode": {"rows": B, "weight_bytes": w_bytes,
                               "lm_head_softcap_fused_us": lm_us[True],
                               "linear_then_soft_cap_us": lm_us[False],
                               "fused_weight_stream_TBps": w_bytes / (lm_us[True] * 1e-6) / 1e12,
                               "speedup": lm_us[False] / lm_us[True],
                               "note": "HIP-graph replays of 3 calls on 3 weight copies (cold in the caches), "
                                       "HIP events"},
            "data": "synthetic: random token ids, weights N(0, 0.02), forget-gate bias 3"}


def load_traffic(kernel, workload):
    """Calibrated HBM bytes per launch of `kernel` on `workload` from profiles/hbm_traffic.json, else None."""
    try:
        with open(TRAFFIC_FILE) as fh:
            rec = json.load(fh)
    except (OSError, ValueError):
        return None
    ent = rec.get("kernels", {}).get(kernel)
    if not ent or ent.get("workload") != workload:
        return None
    return ent.get("hbm_bytes_per_launch")


def _progress(what):
    """One line on stderr per finished entry (stdout carries only the JSON line)."""
    print(f"[bench] {what} done", file=sys.stderr, flush=True)


def summarize_trace(trace_dir, headline_calls):
    """Markdown table of a rocprofv3 --kernel-trace run of this script: calls, mean, min and max
    duration per kernel, and on its own line the headline: the pipelined chunkwise kernel's
    dispatches that follow the 512 MB cache flush and the call's gate prep.  The headline entry's
    first PATTERN_WARM_CALLS such dispatches are its untimed (flush, call) pairs, the next
    `headline_calls` its timed calls (the back-to-back warm-up calls never follow a flush)."""
    import csv
    import glob
    import re
    files = glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit(f"summarize-trace: no *kernel_trace.csv under {trace_dir}")
    rows = []
    for fn in files:
        with open(fn) as fh:
            rows += [(int(r["Start_Timestamp"]), r["Kernel_Name"], (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
                     for r in csv.DictReader(fh)]
    rows.sort()

    def short(name):
        name = name.replace("(anonymous namespace)::", "").replace("xl::fused::pipe::", "")
        name = name.replace("xl::fused::", "").replace("xl::", "")
        name = re.sub(r"\(.*$", "", name)  # drop the parameter list
        return re.sub(r"^void ", "", name)

    per = {}
    head = []
    prev = [("", 0.0), ("", 0.0)]  # the two kernels before this one
    for _, name, us in rows:
        sn = short(name)
        per.setdefault(sn, []).append(us)
        # a timed call: flush fill, then the call's gate prep, then this kernel
        if (sn.startswith(PREFILL_KERNEL + "<bf16_t, 256, false>") and "gate_prep_kernel" in prev[1][0]
                and "FillFunctor<float>" in prev[0][0] and prev[0][1] >= 40.0):
            head.append(us)
        prev = [prev[1], (name, us)]
    warm, head = head[:PATTERN_WARM_CALLS], head[PATTERN_WARM_CALLS:PATTERN_WARM_CALLS + headline_calls]
    print("| kernel | calls | mean us | min us | max us |\n|---|---|---|---|---|")
    if head:
        print(f"| {PREFILL_KERNEL}<bf16_t, 256, false>, the {len(head)} timed cfg2 headline calls (after the cache "
              f"flush) | {len(head)} | {statistics.mean(head):.1f} | {min(head):.1f} | {max(head):.1f} |")
    if warm:
        print(f"| {PREFILL_KERNEL}<bf16_t, 256, false>, the headline's {len(warm)} untimed (flush, call) pairs before "
              f"them | {len(warm)} | {statistics.mean(warm):.1f} | {min(warm):.1f} | {max(warm):.1f} |")
    for name, ts in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        print(f"| {name} | {len(ts)} | {statistics.mean(ts):.1f} | {min(ts):.1f} | {max(ts):.1f} |")


def summarize_pmc(fetch_dir, write_dir):
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of every kernel, scaled by the soft-cap stream's reading.
    Each argument may list several rocprofv3 output directories, comma-separated."""
    import csv
    import glob

    def per_kernel(dirs, counter):
        acc = {}
        files = [fn for d in dirs.split(",") for fn in glob.glob(os.path.join(d, "**", "*counter_collection.csv"),
                                                                  recursive=True)]
        for fn in files:
            with open(fn) as fh:
                for row in csv.DictReader(fh):
                    if row["Counter_Name"] != counter:
                        continue
                    name = row["Kernel_Name"]
                    key = next((k for k in (PREFILL_KERNEL, PREFILL_KERNEL_FUSED, SOFT_CAP_KERNEL, "mlstm_step_kernel",
                                            "gate_prep_kernel",
                                            SLSTM_KERNEL, SEQ_KERNEL, CONV_KERNEL, GROUP_NORM_KERNEL,
                                            RMS_GATE_KERNEL, GATE_PROJ_KERNEL, GATE_ROWS_KERNEL,
                                            LM_HEAD_CFG3_KERNEL, LM_HEAD_CFG4_KERNEL, *BWD_KERNELS)
                                if k in name), None)
                    if key is None:
                        continue
                    acc.setdefault(key, {}).setdefault(row["Dispatch_Id"], 0.0)
                    acc[key][row["Dispatch_Id"]] += float(row["Counter_Value"])  # summed over TCC instances
        # KiB -> bytes; the median dispatch of each kernel, except the calibration stream, whose
        # largest dispatch is the known-size one (smaller soft-cap launches run in other entries)
        return {k: (max(v.values()) if k == SOFT_CAP_KERNEL else statistics.median(v.values())) * 1024
                for k, v in acc.items()}

    fetch, write = per_kernel(fetch_dir, "FETCH_SIZE"), per_kernel(write_dir, "WRITE_SIZE")
    if SOFT_CAP_KERNEL not in fetch or SOFT_CAP_KERNEL not in write:
        raise SystemExit("summarize-pmc: the soft-cap calibration stream is missing from the CSVs")
    sc_bytes = 2 * SOFT_CAP_SHAPE[0] * SOFT_CAP_SHAPE[1] * SOFT_CAP_SHAPE[2]  # read once, written once
    f_scale, w_scale = sc_bytes / fetch[SOFT_CAP_KERNEL], sc_bytes / write[SOFT_CAP_KERNEL]
    from xlstm_hip.workloads import CFG1, CFG2
    wl_slstm, wl_seq = _workloads()
    work = {SLSTM_KERNEL: (wl_slstm, slstm_bytes()), SEQ_KERNEL: (wl_seq, mlstm_sequence_bytes()),
            PREFILL_KERNEL: ("cfg2 mlstm_chunkwise prefill",
                             prefill_bytes(CFG2.B, CFG2.NH, CFG2.S, CFG2.DQK, CFG2.DV)),
            PREFILL_KERNEL_FUSED: ("cfg2 mlstm_chunkwise prefill (fused schedule)",
                                   prefill_bytes(CFG2.B, CFG2.NH, CFG2.S, CFG2.DQK, CFG2.DV)),
            SOFT_CAP_KERNEL: ("cfg3 logit soft_cap (cap 30) [1,2048,50304] bf16", 2 * sc_bytes),
            "mlstm_step_kernel": ("cfg1 mlstm decode step", decode_bytes(CFG1.B, CFG1.NH, CFG1.DQK, CFG1.DV)),
            # gate prep: reads i, f (bf16), writes 258 floats of per-chunk gate scans per 64 tokens
            "gate_prep_kernel": ("cfg2 chunkwise gate prep",
                                 2 * CFG2.B * CFG2.NH * CFG2.S * 2 + CFG2.B * CFG2.NH * (CFG2.S // 64) * 258 * 4),
            **layer_stage_work()}
    # the fused path's launches keep C and dC packed (3 bytes a value), the two-pass ones float32
    bwb = bwd_kernel_bytes(CFG2.B, CFG2.NH, CFG2.S, CFG2.DQK, CFG2.DV, 64)
    bwp = bwd_kernel_bytes(CFG2.B, CFG2.NH, CFG2.S, CFG2.DQK, CFG2.DV, 64, st_esz=3)
    for k, short in BWD_KERNELS.items():
        work[k] = (f"cfg2 chunkwise backward: {short}", (bwp if short in FUSED_PATH else bwb)[short])
    out = {"calibration": {"kernel": SOFT_CAP_KERNEL, "bytes_read": sc_bytes, "bytes_written": sc_bytes,
                           "fetch_scale": f_scale, "write_scale": w_scale},
           "kernels": {}}
    for k in sorted(set(fetch) & set(write)):
        rd, wr = fetch[k] * f_scale, write[k] * w_scale
        out["kernels"][k] = {"workload": work[k][0], "fetch_bytes": rd, "write_bytes": wr,
                             "hbm_bytes_per_launch": rd + wr, "algorithmic_bytes": work[k][1],
                             "ratio_to_algorithmic": (rd + wr) / work[k][1],
                             "raw_fetch_kib": fetch[k] / 1024, "raw_write_kib": write[k] / 1024}
    print(json.dumps(out, indent=1))


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _blas() -> str:
    """The BLAS torch was built with and, where torch names it, the library version."""
    import re
    cfg = torch.__config__.show()
    blas = re.search(r"BLAS_INFO=([^,\s]+)", cfg)
    ver = re.search(r"(Intel\(R\) [^\n]*Math Kernel Library[^\n]*)", cfg)
    out = blas.group(1) if blas else "unknown"
    return f"{out} ({ver.group(1).strip()})" if ver else out


def bench_cfg0(args, dev):
    """BASELINE config 0 on the GPU: one float32 mlstm_chunkwise call (B1 NH8 S256 DQK256 DV512, L 64,
    last states returned): the two-pass algorithm, states on float32 MFMA, outputs on bf16 MFMA in the
    three-product form; replayed from a HIP graph, HIP events."""
    import xlstm_hip
    from xlstm_hip.workloads import CFG0, chunkwise_inputs
    x = chunkwise_inputs(CFG0, device=dev)
    t = _timed(lambda: xlstm_hip.mlstm_chunkwise(*x, return_last_states=True, chunk_size=CFG0.L), dev,
               max(20, args.steps))
    return {"workload": "cfg0 mlstm_chunkwise fp32 B1 NH8 S256 DQK256 DV512 L64", "us_per_call": 1e3 * t["ms"],
            "us_min": 1e3 * t["ms_min"], "mode": t["mode"], "algo": "two_pass (states: float32 MFMA; outputs: bf16 MFMA, three products)"}


def cpu_baseline(args):
    """Oracle (torch on the host) on bounded samples: cfg2 prefill tokens/s (the headline's unit),
    cfg0 us per call, cfg1 decode us per step."""
    from oracle import mlstm as om
    from xlstm_hip.workloads import CFG0, CFG1, CFG2, chunkwise_inputs, step_inputs
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    # prefill sample: batch row 0 of cfg2 (all 8 heads, full S; bf16 inputs upcast, fp32 states)
    S = CFG2.S
    x = tuple(t.float() for t in chunkwise_inputs(CFG2, B=1))
    om.mlstm_chunkwise(*x, return_last_states=True, chunk_size=args.chunk_size)  # warm-up
    reps, t0 = 0, time.perf_counter()
    while reps < 3 or (time.perf_counter() - t0 < 10.0 and reps < 50):
        om.mlstm_chunkwise(*x, return_last_states=True, chunk_size=args.chunk_size)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    pre_tps = S / dt
    # cfg0: the whole config, >= 20 reps, median
    x0 = chunkwise_inputs(CFG0)
    for _ in range(2):
        om.mlstm_chunkwise(*x0, return_last_states=True, chunk_size=CFG0.L)
    c0 = []
    while len(c0) < 20:
        t1 = time.perf_counter()
        om.mlstm_chunkwise(*x0, return_last_states=True, chunk_size=CFG0.L)
        c0.append(time.perf_counter() - t1)
    # decode sample: cfg1 step, 100 chained steps (the 1000-step figure is this rate x 1000)
    q, k, v, i, f, C, n, m = step_inputs(CFG1)
    om.mlstm_recurrent_step(q, k, v, i, f, C, n, m)
    t0 = time.perf_counter()
    nst = 100
    for _ in range(nst):
        _, (C, n, m) = om.mlstm_recurrent_step(q, k, v, i, f, C, n, m)
    dec_us = 1e6 * (time.perf_counter() - t0) / nst
    return {
        "value": pre_tps, "unit": "tokens/s", "cores": cores, "kind": "port",
        "cpu_model": _cpu_model(), "blas": _blas(), "torch": torch.__version__,
        "sample": f"oracle.mlstm.mlstm_chunkwise (torch {torch.__version__} CPU, fp32, {cores} threads) on cfg2 "
                  f"batch row 0, 8 heads, S={S}, L={args.chunk_size}: {reps} reps, {dt * 1e3:.1f} ms each",
        "cfg0_us_per_call": 1e6 * statistics.median(c0),
        "cfg0_sample": "oracle.mlstm.mlstm_chunkwise on all of cfg0 (fp32 B1 NH8 S256 DQK256 DV512 L64, last "
                       "states), 20 reps after 2 warm-ups, median",
        "decode_us_per_step": dec_us,
        "decode_sample": f"oracle.mlstm.mlstm_recurrent_step on cfg1, {nst} chained steps after 1 warm-up (1000 "
                         f"steps extrapolate to {dec_us * 1e-3:.0f} ms)",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--warmup-seconds", type=float, default=1.0,
                    help="after --warmup calls, keep calling (untimed) for this long so the clocks settle")
    ap.add_argument("--chunk-size", type=int, default=64)
    ap.add_argument("--algo", default="auto", choices=["auto", "pipelined", "fused", "two_pass"])
    ap.add_argument("--decode-steps", type=int, default=1000)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-soft-cap", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the sLSTM, recurrent-sequence and any-S entries")
    ap.add_argument("--no-stacks", action="store_true", help="skip the config 3 / 4 end-to-end stacks")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"))
    ap.add_argument("--summarize-trace", metavar="TRACE_DIR",
                    help="per-kernel durations of a rocprofv3 --kernel-trace run of this script (no GPU)")
    args = ap.parse_args()
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc)
        return
    if args.summarize_trace:
        summarize_trace(args.summarize_trace, args.steps)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on ONE GPU only (no collectives); use --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    import xlstm_hip
    xlstm_hip.load_library()

    pre = bench_prefill(args, dev)
    _progress("prefill")
    cfg = pre["cfg"]
    value = pre["tokens"] / (pre["ms"] * 1e-3)
    tflops = pre["flops"] / (pre["ms"] * 1e-3) / 1e12
    gbs = pre["bytes"] / (pre["ms"] * 1e-3) / 1e9
    out = {
        "metric": "mLSTM chunkwise prefill tokens/s (7B heads) + decode step us; % roofline",
        "value": value, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": pre["ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded N(0,1) inputs of BASELINE config 2)",
        "config": {"workload": "cfg2 mlstm_chunkwise prefill", "B": cfg.B, "NH": cfg.NH, "S": cfg.S,
                   "DQK": cfg.DQK, "DV": cfg.DV, "chunk_size": pre["L"], "states": "fp32",
                   "return_last_states": True, "algo": args.algo},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": tflops / PEAK_BF16_TFLOPS,
                     "traffic": load_traffic(PREFILL_KERNEL, "cfg2 mlstm_chunkwise prefill")
                     if (pre["L"] == 64 and args.algo in ("auto", "pipelined")) else None,
                     "flops_per_call": pre["flops"],
                     "timing": f"HIP events per call ({pre['mode']}), caches flushed"},
        "roofline_hbm": {"achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                         "bytes_per_call": pre["bytes"]},
        "prefill_ms_median": pre["ms_median"], "prefill_ms_min": pre["ms_min"], "prefill_wall_ms": pre["wall_ms"],
        "prefill_ms_graph": pre["ms_graph"],
    }
    if pre["L"] == 64 and args.algo == "auto":
        pf = bench_prefill(args, dev, steps=max(3, args.steps // 2), algo="fused")
        out["prefill_fused"] = {"ms_per_call": pf["ms"], "tokens_per_s": pf["tokens"] / (pf["ms"] * 1e-3),
                                "tflops": pf["flops"] / (pf["ms"] * 1e-3) / 1e12}
        # cfg2's chunk_size 128 sweep: the same single-pass kernel (64-token chunks; the forward is
        # chunk-size invariant), so its TFLOP/s are counted with the 64-token algorithm it runs
        p128 = bench_prefill(args, dev, L=128, steps=max(3, args.steps // 4))
        fl64 = prefill_flops(cfg.B, cfg.NH, cfg.S, cfg.DQK, cfg.DV, 64)
        out["prefill_chunk_size_128"] = {
            "ms_per_call": p128["ms"], "tokens_per_s": p128["tokens"] / (p128["ms"] * 1e-3),
            "tflops_64_token_algorithm": fl64 / (p128["ms"] * 1e-3) / 1e12,
            "flops_per_call_reference_L128": p128["flops"]}
    if not args.no_decode:
        dec = bench_decode(args, dev)
        _progress("decode")
        dgbs = dec["bytes"] / (dec["us_per_step"] * 1e-6) / 1e9
        out["decode"] = {"workload": "cfg1 mlstm decode step", "us_per_step": dec["us_per_step"],
                         "tokens_per_s": dec["cfg"].B / (dec["us_per_step"] * 1e-6), "steps": dec["steps"],
                         "mode": dec["mode"], "state_sets": dec["state_sets"],
                         "roofline": {"bound": "hbm", "achieved": dgbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                      "frac": dgbs / PEAK_HBM_GBS, "bytes_per_step": dec["bytes"],
                                      "traffic": load_traffic("mlstm_step_kernel", "cfg1 mlstm decode step")},
                         "copy_ceiling": {"what": "xl_mlstm_step_copy_ceiling: each step's C copied in place "
                                                  "with the step's grid, thread map and 16-byte nontemporal "
                                                  "loads/stores and nothing else (same 6-set rotation, HIP "
                                                  "graph)", "bytes": dec["copy_bytes"],
                                          "us": dec["copy_us"],
                                          "step_fraction_of_copy": dec["copy_us"] / dec["us_per_step"]}}
    if not args.no_soft_cap:
        out["soft_cap"] = bench_soft_cap(args, dev)
        _progress("soft_cap")
    if not args.no_extra:
        out["slstm_sequence"] = bench_slstm_sequence(args, dev)
        _progress("slstm_sequence")
        out["slstm_step"] = bench_slstm_step(args, dev)
        _progress("slstm_step")
        out["mlstm_sequence"] = bench_mlstm_sequence(args, dev)
        _progress("mlstm_sequence")
        out["arbitrary_length"] = bench_arbitrary_length(args, dev)
        _progress("arbitrary_length")
        out["cfg3_heads_chunkwise"] = bench_cfg3_heads(args, dev)
        _progress("cfg3_heads_chunkwise")
        out["slstm_conv1d_silu"] = bench_slstm_conv(args, dev)
        _progress("slstm_conv1d_silu")
        out["slstm_group_norm"] = bench_group_norm(args, dev)
        _progress("slstm_group_norm")
        out["mlstm_output_gate"] = bench_mlstm_output_gate(args, dev)
        _progress("mlstm_output_gate")
        out["slstm_gate_proj"] = bench_gate_proj(args, dev)
        _progress("slstm_gate_proj")
        out["chunkwise_bwd"] = bench_chunkwise_bwd(args, dev)
        _progress("chunkwise_bwd")
    if not args.no_extra:
        out["cfg0"] = bench_cfg0(args, dev)
        _progress("cfg0")
    if not args.no_stacks:
        out["cfg3_stack"] = bench_stack(args, dev, "cfg3")
        _progress("cfg3_stack")
        out["cfg4_stack"] = bench_stack(args, dev, "cfg4")
        _progress("cfg4_stack")
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args)
        _progress("cpu_baseline")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
