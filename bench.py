#!/usr/bin/env python3
"""W4A16 SwiGLU FFN benchmark on one MI355X: decode GB/s and prefill TFLOP/s at the Llama-3-8B FFN shape.

Headline `value`: Llama-3-8B FFN layer decode, M = 1, fp16 activations, W4A16 group 128,
as algorithmic GB/s (weights + x + y per layer, inputs resident in HBM). A step is one FFN layer pass over one
batch. 32 independent weight sets rotate (2.95 GB, the FFN layers of one Llama-3-8B), so neither a layer nor the 32
matrices of any one projection fit in the 256 MB Infinity Cache.
The timed steps are eager C ABI calls (one hm_ffn_forward per step, as the reference's model loop calls its
operators); the host enqueues faster than the GPU runs them. extra.decode_M1_event_median_us is the same pass in graphs
of 48 timed with HIP events, and extra.decode_M1_eager adds the host time per call and the reference-signature
GpuFfnModel::forward's. Also reported: decode M = 4 and 16, prefill M = 512 and 2048 (TFLOP/s; 8 weight sets rotate, 738 MB),
a 32-layer decode stack with
RMSNorm and residual between layers, the Qwen2.5-14B g = 64 shape, the roofline of the headline step's two kernels
and of the prefill gate_up GEMM measured with HIP events, and the reference CPU path (restated AVX-512 GEMV) timed on
this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick]
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0           # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0   # MI355X dense fp16 / bf16 MFMA
PREFILL_SETS = 8                # weight sets a prefill graph rotates: 8 Llama-3-8B layers are 738 MB, their gate_up 470 MB


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def ffn_bytes(m, h, i, g):
    """Algorithmic bytes of one FFN layer: int4 weights + 2-byte scale + 1-byte zero per group, x in, y out."""
    w = 3 * (h * i // 2 + (h * i // g) * 3)
    return w + m * h * 2 + m * h * 2


def ffn_flops(m, h, i):
    return 2 * m * h * i * 3


def make_layers(hm, torch, dev, h, i, g, count, dtype=None, seed=0):
    dtype = dtype or torch.float16
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    layers = []
    for _ in range(count):
        mats = []
        for k, n in ((h, i), (h, i), (i, h)):
            q = torch.randint(0, 16, (k, n), dtype=torch.uint8, device=dev, generator=gen)
            s = (torch.rand((k // g, n), device=dev, generator=gen) * 0.019 + 0.001).to(dtype)
            z = torch.randint(0, 16, (k // g, n), dtype=torch.uint8, device=dev, generator=gen)
            mats.append((q, s, z))
        layers.append(hm.FfnLayer.from_logical(*mats, g, dtype=dtype))
        del mats
    torch.cuda.synchronize()
    return layers


def qkv_bench(hm, torch, dev, h, g, sets=24):
    """Q, K, V projections of one attention block: three launches against one on the concatenated matrix."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    widths = (h, h // 4, h // 4)
    parts, fused = [], []
    for _ in range(sets):
        mats = []
        for n in widths:
            q = torch.randint(0, 16, (h, n), dtype=torch.uint8, device=dev, generator=gen)
            s = (torch.rand((h // g, n), device=dev, generator=gen) * 0.019 + 0.001).to(torch.float16)
            z = torch.randint(0, 16, (h // g, n), dtype=torch.uint8, device=dev, generator=gen)
            mats.append(hm.RepackedMatrix.from_logical(q, s, z, g, dtype=torch.float16))
        parts.append(mats)
        fused.append(hm.RepackedMatrix.concat(mats))
    torch.cuda.synchronize()
    n_all = sum(widths)
    out = {}
    for m, count in ((1, sets), (2048, sets)):
        x = torch.randn((m, h), device=dev).to(torch.float16)
        y = torch.empty((m, n_all), device=dev, dtype=torch.float16)
        ws = torch.empty(max(parts[0][0].workspace_bytes(m), fused[0].workspace_bytes(m)) + 512, dtype=torch.uint8, device=dev)

        def separate():
            for mats in parts[:count]:
                c0 = 0
                for w in mats:
                    hm.packed_linear(y[:, c0:c0 + w.n], x, w, workspace=ws)
                    c0 += w.n

        def one():
            for w in fused[:count]:
                hm.packed_linear(y, x, w, workspace=ws)

        t_sep = time_graph(torch, graph_of(torch, separate), 20, 0.3, 2) / count
        t_one = time_graph(torch, graph_of(torch, one), 20, 0.3, 2) / count
        if m == 1:
            b = h * n_all // 2 + (h // g) * n_all * 3
            out["decode_M1"] = {"us_three_launches": round(t_sep * 1e6, 2), "us_one_launch": round(t_one * 1e6, 2),
                                "GB_s_one_launch": round(b / t_one / 1e9, 1)}
        else:
            f = 2.0 * m * h * n_all
            out[f"prefill_M{m}"] = {"us_three_launches": round(t_sep * 1e6, 1), "us_one_launch": round(t_one * 1e6, 1),
                                    "TFLOP_s_one_launch": round(f / t_one / 1e12, 1)}
    return out


def ksplit_bench(hm, torch, dev, h, inter, g, sets=12):
    """The down projection kept as a K-split pair (two [inter/2, h] matrices, both shares on the GPU, the second
    adding into the output) against the same projection as one [inter, h] matrix."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    k0 = inter // 2

    def mat(k):
        q = torch.randint(0, 16, (k, h), dtype=torch.uint8, device=dev, generator=gen)
        s = (torch.rand((k // g, h), device=dev, generator=gen) * 0.019 + 0.001).to(torch.float16)
        z = torch.randint(0, 16, (k // g, h), dtype=torch.uint8, device=dev, generator=gen)
        return hm.RepackedMatrix.from_logical(q, s, z, g, dtype=torch.float16)

    pairs = [(mat(k0), mat(inter - k0)) for _ in range(sets)]
    whole = [mat(inter) for _ in range(sets)]
    torch.cuda.synchronize()
    out = {}
    for m, count in ((1, sets), (2048, min(sets, PREFILL_SETS))):
        act = torch.randn((m, inter), device=dev).to(torch.float16)
        y = torch.empty((m, h), device=dev, dtype=torch.float16)
        ws = torch.empty(max(whole[0].workspace_bytes(m), 64 << 20) + 512, dtype=torch.uint8, device=dev)

        def split():
            for w0, w1 in pairs[:count]:
                hm.packed_linear_k_split(y, act, w0, w1, workspace=ws)

        def one():
            for w in whole[:count]:
                hm.packed_linear(y, act, w, workspace=ws)

        t_split = time_graph(torch, graph_of(torch, split), 20, 0.3, 2) / count
        t_one = time_graph(torch, graph_of(torch, one), 20, 0.3, 2) / count
        if m == 1:
            b = inter * h // 2 + (inter // g) * h * 3
            out["decode_M1"] = {"us_k_split_pair": round(t_split * 1e6, 2), "us_one_matrix": round(t_one * 1e6, 2),
                                "GB_s_k_split_pair": round(b / t_split / 1e9, 1)}
        else:
            f = 2.0 * m * h * inter
            out[f"prefill_M{m}"] = {"us_k_split_pair": round(t_split * 1e6, 1), "us_one_matrix": round(t_one * 1e6, 1),
                                    "TFLOP_s_k_split_pair": round(f / t_split / 1e12, 1)}
    return out


def graph_of(torch, fn):
    """Captures fn() (enqueueing on the current stream) into a HIP graph after one eager warm-up call."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, replays, warm_seconds=0.0, warm_replays=2):
    """Wall time per replay (barrier + synchronize on both sides), after warm-up replays."""
    for _ in range(warm_replays):
        g.replay()
    torch.cuda.synchronize()
    t_end = time.perf_counter() + warm_seconds
    while time.perf_counter() < t_end:
        g.replay()
        torch.cuda.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(replays):
        g.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / replays


def event_time_graph(torch, g, replays):
    """HIP-event time per replay on the stream the graph runs on (torch replays a graph on the current stream):
    the median over `replays` replays, each bracketed by its own pair of events."""
    g.replay()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(replays)]
    for a, b in evs:
        a.record()
        g.replay()
        b.record()
    torch.cuda.synchronize()
    times = sorted(a.elapsed_time(b) / 1e3 for a, b in evs)
    return times[len(times) // 2]


BLOCK = 48  # layer passes per event-timed block: a decoder replays a model's layers per token


def forward_calls(layers, x, y, ws, stream):
    """One prepared hm_ffn_forward call per weight set (ctypes, all arguments converted once), as a C++ caller of the
    C ABI makes them: the layer's whole channel range, x and y rows of the layer's width."""
    import ctypes

    from heteromega_amd import _lib

    fwd = _lib.load().hm_ffn_forward
    off = (-ws.data_ptr()) % 256  # the C ABI takes a 256-byte aligned workspace
    m, h = x.shape
    calls = []
    for L in layers:
        a = (L._h, ctypes.c_void_p(y.data_ptr()), y.stride(0), ctypes.c_void_p(x.data_ptr()), x.stride(0), m, 0, L.inter,
             ctypes.c_void_p(ws.data_ptr() + off), ws.numel() - off, ctypes.c_void_p(stream))
        calls.append(a)

    def run(count):
        for i in range(count):
            rc = fwd(*calls[i % len(calls)])
            if rc != 0:
                raise RuntimeError(_lib.last_error())
    return run


def decode_bench(hm, torch, dev, layers, m, h, steps, warmup, warm_seconds=0.0, blocks=0):
    """Seconds per decode step (one FFN layer pass), cycling through the weight sets.

    The timed region is exactly `steps` passes enqueued as eager C ABI calls (hm_ffn_forward, one call per step as the
    reference's model loop calls its operators), wall-clocked with a synchronize on both sides, after `warmup` untimed
    passes, warm_seconds of untimed graph replays (the clock settles) and one untimed run of the same `steps` passes.
    Eager enqueueing (6 us of host time per call) stays ahead of the GPU (20 us per pass), and its fixed cost per timed
    region is below a graph replay's (at 20 steps 20.9 against 21.3 us per pass; equal at 240). With blocks > 0 also
    the median per pass over `blocks` event-timed replays of a graph of BLOCK passes (the benchmark protocol's method:
    HIP events, median). Returns (wall seconds per step, median seconds per step or None, graph of BLOCK passes, buffers)."""
    x = torch.randn((m, h), device=dev).to(layers[0].dtype)
    y = torch.empty_like(x)
    ws = layers[0].workspace(m)
    sets = len(layers)

    def run(count):
        def fn():
            for i in range(count):
                layers[i % sets].forward(x, y, workspace=ws)
        return fn

    g_block = graph_of(torch, run(BLOCK))
    eager = forward_calls(layers, x, y, ws, torch.cuda.current_stream().cuda_stream)
    eager(warmup)
    torch.cuda.synchronize()
    t_end = time.perf_counter() + warm_seconds
    while time.perf_counter() < t_end:
        g_block.replay()
        torch.cuda.synchronize()
    eager(steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    eager(steps)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    median = event_time_graph(torch, g_block, blocks) / BLOCK if blocks > 0 else None
    assert bool(torch.isfinite(y).all()), "decode output is not finite"
    return wall, median, g_block, (x, y, ws)


def prefill_bench(hm, torch, dev, layers, m, h, steps, warmup):
    """Seconds per prefill layer: replays of a graph of one layer pass on each of PREFILL_SETS weight sets (so the
    256 MB Infinity Cache cannot hold the weights between passes), after half a second of untimed replays (the
    part's clock settles under sustained MFMA load); the median of event-timed replays."""
    x = torch.randn((m, h), device=dev).to(layers[0].dtype)
    y = torch.empty_like(x)
    ws = layers[0].workspace(m)
    sets = layers[:PREFILL_SETS]

    def run():
        for L in sets:
            L.forward(x, y, workspace=ws)

    g = graph_of(torch, run)
    time_graph(torch, g, 1, 0.5, max(1, warmup // 2))
    sec = event_time_graph(torch, g, max(3, steps // 2))
    assert bool(torch.isfinite(y).all()), "prefill output is not finite"
    return sec / len(sets)


def prefill_gate_up_roofline(hm, torch, dev, layers, m, h, i, replays):
    """The fused gate_up GEMM (SwiGLU epilogue) at m rows: median event time per launch over graphs of one launch on
    each of PREFILL_SETS weight sets, against the dense fp16 MFMA peak."""
    x = torch.randn((m, h), device=dev).to(layers[0].dtype)
    act = torch.empty((m, i), dtype=layers[0].dtype, device=dev)
    sets = layers[:PREFILL_SETS]

    def run():
        for L in sets:
            L.gate_up(x, act)

    g = graph_of(torch, run)
    time_graph(torch, g, 1, 0.5, 2)
    sec = event_time_graph(torch, g, replays) / len(sets)
    flops = 2.0 * m * h * 2 * i
    achieved = flops / sec / 1e12
    return {"kernel": "gemm_kernel<F16, 128, true, 8, 2, 8, 4, 2> (fused gate_up + SwiGLU, 128 x 256 tiles, one barrier per two K tiles)", "bound": "mfma",
            "achieved": round(achieved, 1), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4),
            "traffic": measured_traffic(PREFILL_TRAFFIC, "traffic_bytes_per_launch"), "avg_launch_us": round(sec * 1e6, 2),
            "algorithmic_flops_per_launch": int(flops), "rows": m,
            "timing": f"median of {replays} event-timed replays of a graph of {len(sets)} launches ({len(sets)} weight sets), after 0.5 s of untimed replays"}


def eager_bench(hm, torch, dev, layers, h, inter, calls=480):
    """The headline layer called eagerly (no graph): hm_ffn_forward through ctypes with prepared arguments, over the
    rotating weight sets. Returns (GPU us per layer from HIP events around the enqueues, host us per call)."""
    from heteromega_amd import _lib
    import ctypes

    L = _lib.load()
    x = torch.randn((1, h), device=dev).to(layers[0].dtype)
    y = torch.empty_like(x)
    ws = layers[0].workspace(1)
    off = (-ws.data_ptr()) % 256  # the C ABI takes a 256-byte aligned workspace
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [(Lr._h, ctypes.c_void_p(y.data_ptr()), h, ctypes.c_void_p(x.data_ptr()), h, 1, 0, inter, ctypes.c_void_p(ws.data_ptr() + off),
             ws.numel() - off, stream) for Lr in layers]
    fwd = L.hm_ffn_forward
    for i in range(2 * len(args)):
        assert fwd(*args[i % len(args)]) == 0
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = None
    for _ in range(3):
        e0.record()
        t0 = time.perf_counter()
        for i in range(calls):
            fwd(*args[i % len(args)])
        host = (time.perf_counter() - t0) / calls
        e1.record()
        torch.cuda.synchronize()
        gpu = e0.elapsed_time(e1) / 1e3 / calls
        if best is None or gpu < best[0]:
            best = (gpu, host)
    assert bool(torch.isfinite(y).all()), "eager decode output is not finite"
    return best[0] * 1e6, best[1] * 1e6


def shim_eager_host_us(hm, torch, dev, h, inter, calls=200):
    """Host us per call of the reference-signature heteromega::GpuFfnModel::forward (bf16, M = 1) on one layer packed
    from host tiles: the C++ operator surface a reference caller links, reached here through its pybind module."""
    import numpy as np
    from heteromega_amd import _reference_shim as shim

    rng = np.random.default_rng(5)

    def tiles(k, n):
        q = rng.integers(0, 16, (k, n), dtype=np.uint8)
        s = (rng.uniform(0.001, 0.02, (k // 128, n)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        z = rng.integers(0, 16, (k // 128, n), dtype=np.int8)
        return torch.from_numpy(hm.pack_w4a16(q, s, z)).to(dev)

    model = shim.GpuFfnModel()
    model.add_layer(tiles(h, inter), tiles(h, inter), tiles(inter, h), h, inter)
    x = torch.randn((1, h), device=dev).to(torch.bfloat16)
    y = torch.empty_like(x)
    st = torch.cuda.current_stream().cuda_stream
    for _ in range(10):
        model.forward(0, x, y, st)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(calls):
        model.forward(0, x, y, st)
    host = (time.perf_counter() - t0) / calls
    torch.cuda.synchronize()
    return host * 1e6


DECODE_TRAFFIC = os.path.join(ROOT, "profiles", "pmc_gemv_gate_up_llama8b_decode_m1.md")
PREFILL_TRAFFIC = os.path.join(ROOT, "profiles", "pmc_gemm_gate_up_llama8b_prefill_m2048.md")


def measured_traffic(path, key):
    """HBM bytes of one launch (or step) from a committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (calibrated there
    against a copy kernel of known size): the integer after `key:`, or None without one."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return int(line.split(":", 1)[1].strip())
    except (OSError, ValueError):
        pass
    return None


def calibration_copy(torch, dev):
    """A plain copy kernel of known size for the rocprofv3 --pmc passes: 8 launches that read and write 64 MiB each
    (torch bitwise_not over int32, four buffers the Infinity Cache cannot hold)."""
    words = (64 << 20) // 4
    bufs = [torch.empty(words, dtype=torch.int32, device=dev).random_(0, 1 << 30) for _ in range(4)]
    outs = [torch.empty_like(b) for b in bufs]
    torch.cuda.synchronize()
    for r in range(8):
        torch.bitwise_not(bufs[r % 4], out=outs[r % 4])
    torch.cuda.synchronize()
    log(f"pmc probe: 8 copy launches of {words * 4} bytes read + {words * 4} bytes written")


def pmc_probe(hm, torch, dev, H, I, G, sets, rows=1):
    """Eager launches for one rocprofv3 --pmc pass: a copy kernel of known size (calibration), then the fused
    gate_up GEMV and the down GEMV of the headline workload (or of the same layer at `rows` rows), then the layer's
    forward (whose one-row kernels are the pair-unit builds), on rotating weight sets."""
    calibration_copy(torch, dev)
    layers = make_layers(hm, torch, dev, H, I, G, sets)
    x = torch.randn((rows, H), device=dev).to(torch.float16)
    act = torch.empty((rows, I), dtype=torch.float16, device=dev)
    y = torch.empty((rows, H), dtype=torch.float16, device=dev)
    for r in range(2 * sets):
        layers[r % sets].gate_up(x, act)
    torch.cuda.synchronize()
    log(f"pmc probe: {2 * sets} gate_up launches (M={rows})")
    for r in range(2 * sets):
        layers[r % sets].down(act, y)
    torch.cuda.synchronize()
    log(f"pmc probe: {2 * sets} down launches (M={rows})")
    ws = layers[0].workspace(rows)
    for r in range(2 * sets):
        layers[r % sets].forward(x, y, workspace=ws)
    torch.cuda.synchronize()
    log(f"pmc probe: {2 * sets} layer forwards (M={rows}; at one row the pair-unit gate_up and the down GEMV that "
        f"forms its split pairs)")


def host_cpus():
    """(usable logical CPUs, physical cores among them, CPU model) of this process's CPU set."""
    usable = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
    cores = set()
    for c in usable:
        try:
            with open(f"/sys/devices/system/cpu/cpu{c}/topology/core_id") as f:
                core = f.read().strip()
            with open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id") as f:
                pkg = f.read().strip()
            cores.add((pkg, core))
        except OSError:
            cores.add(("?", str(c)))
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return len(usable), len(cores), model


def cpu_baseline(seconds, h, i, label):
    """The reference CPU decode FFN (restated AVX-512 GEMV on 4352-byte tiles, bf16, M = 1) on this host, as the
    reference times its CPU kernel (test_layout_cpu.cpp:15-44, :153-183): 20 warm-up calls, then timed calls, over a
    thread sweep from 1 to the physical cores; the best is reported."""
    import numpy as np

    from oracle import oracle as o

    rng = np.random.default_rng(0)

    def tiles(k, n):
        t = (k // 128) * (n // 64)
        a = rng.integers(0, 256, (t, 4352), dtype=np.uint8)
        a[:, 4096:4224] = o.bf16_bits(rng.uniform(0.001, 0.02, (t, 64)).astype(np.float32)).view(np.uint8).reshape(t, 128)
        zr = rng.integers(0, 16, (t, 8, 8), dtype=np.uint8)
        a[:, 4224:] = np.repeat(zr, 2, axis=1).reshape(t, 128)
        return np.ascontiguousarray(a.reshape(-1))

    gate, up, down = tiles(h, i), tiles(h, i), tiles(i, h)
    x = o.bf16_bits(rng.standard_normal(h).astype(np.float32))
    scratch, y = np.empty(2 * i, np.uint16), np.empty(h, np.uint16)
    logical, physical, model = host_cpus()
    sweep = sorted({t for t in (1, 2, 4, 8, 16, 32, 64, 128) if t < physical} | {physical})
    nbytes = ffn_bytes(1, h, i, 128)
    results = {}
    branch = 0
    budget = seconds / len(sweep)
    for th in sweep:
        for _ in range(20):
            _, branch = o.cpu_ffn_decode(x, gate, up, down, h, i, th, -1, scratch, y)
        n, t0 = 0, time.perf_counter()
        while True:
            o.cpu_ffn_decode(x, gate, up, down, h, i, th, -1, scratch, y)
            n += 1
            el = time.perf_counter() - t0
            if n >= 100 or el > budget:
                break
        results[th] = (el / n, n)
    best_th = min(results, key=lambda t: results[t][0])
    sec, n = results[best_th]
    return {
        "value": round(nbytes / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": best_th,
        "kind": "port",
        "sample": f"{label} FFN decode M=1 (gate, up, silu_*mul_, down GEMVs on 4352-B tiles, bf16), {n} timed calls after 20 warm-ups "
                  f"at the best of {len(sweep)} thread counts 1..{physical}: {best_th} threads ({'AVX-512' if branch else 'scalar'} branch, "
                  f"restated reference w4a16_gemv_cpu_fused_packed), CPU {model}, {physical} physical cores in this process's "
                  f"CPU set ({logical} logical CPUs)",
        "ms_per_call": round(sec * 1e3, 3),
        "per_threads_ms": {str(t): round(v[0] * 1e3, 3) for t, v in results.items()},
        "physical_cores": physical,
        "logical_cpus": logical,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=24)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--quick", action="store_true", help="headline decode only")
    ap.add_argument("--sets", type=int, default=32, help="weight sets rotated per decode step (32: one Llama-3-8B's FFN layers)")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="only launch the calibration copy and the headline GEMVs (for rocprofv3 --pmc passes)")
    ap.add_argument("--rows", type=int, default=1, help="rows (M) of the --pmc-probe GEMVs")
    ap.add_argument("--pmc-probe-prefill", action="store_true",
                    help="only launch the fused gate_up GEMM at M=2048 (for rocprofv3 --pmc passes)")
    ap.add_argument("--profile", choices=("decode", "roofline_prefill", "gate_up"),
                    help="only the headline decode steps (the decode roofline's measurement), only the prefill roofline's "
                         "graphs, or only the graphs of the whole-pair gate_up GEMV alone (for rocprofv3 kernel traces)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs the FFN on a single MI355X and has no multi-GPU path "
              f"(--gpus {args.gpus} requested). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    import heteromega_amd as hm

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    H, I, G = 4096, 14336, 128
    out = {}

    if args.pmc_probe:
        pmc_probe(hm, torch, dev, H, I, G, args.sets, args.rows)
        return
    if args.pmc_probe_prefill:
        calibration_copy(torch, dev)
        pl = make_layers(hm, torch, dev, H, I, G, 2)
        xp = torch.randn((2048, H), device=dev).to(torch.float16)
        ap_ = torch.empty((2048, I), dtype=torch.float16, device=dev)
        for r in range(6):
            pl[r % 2].gate_up(xp, ap_)
        torch.cuda.synchronize()
        log("pmc probe: 6 fused gate_up GEMM launches (M=2048)")
        return

    log("building weight sets ...")
    layers = make_layers(hm, torch, dev, H, I, G, args.sets)

    if args.profile == "roofline_prefill":
        rp = prefill_gate_up_roofline(hm, torch, dev, layers, 2048, H, I, 10)
        print(json.dumps({"roofline_prefill": rp}), flush=True)
        return

    # Headline: decode M = 1.
    nbytes = ffn_bytes(1, H, I, G)
    if args.profile != "gate_up":
        sec, med, g1, keep = decode_bench(hm, torch, dev, layers, 1, H, args.steps, args.warmup, warm_seconds=2.0, blocks=40)
        value = nbytes / sec / 1e9
        log(f"decode M=1: {sec * 1e6:.2f} us/layer, {value:.1f} GB/s ({100 * value / HBM_PEAK_GBS:.1f}% of HBM peak); "
            f"event median {med * 1e6:.2f} us/layer")
        # Roofline of the step's kernels: the headline step is hm_ffn_forward at one row, two launches that both stream
        # weights from HBM (the pair-unit gate_up + SwiGLU GEMV, then the down GEMV that forms the pairs two workgroups
        # share); together they move the layer's algorithmic bytes. Timed with HIP events on the stream the graph
        # replays on: the median over 40 replays of a graph of BLOCK back-to-back layer passes, per pass.
        achieved = nbytes / med / 1e9
        out["roofline"] = {
            "kernel": "gemv_kernel<F16, 1, 128, 2, true, 1024, 4, 1> (gate_up + SwiGLU by pair units) + gemv_kernel<F16, 1, 128, 1, false, 512, 4, 2> "
                      "(down, forming the split pairs): the two launches of one headline step (hm_ffn_forward, M=1)",
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(DECODE_TRAFFIC, "traffic_bytes_per_layer_forward"), "avg_launch_us": round(med * 1e6, 3),
            "algorithmic_bytes_per_launch": nbytes,
            "timing": f"per layer pass (both launches): median of 40 event-timed replays of a graph of {BLOCK} passes"}
        if args.profile == "decode":
            print(json.dumps({"decode_us": round(sec * 1e6, 3), "decode_event_median_us": round(med * 1e6, 3), "roofline": out["roofline"]}),
                  flush=True)
            return

    # The whole-pair fused gate_up GEMV alone (what hm_ffn_gate_up launches), with HIP events on the stream its graph
    # replays on: the median over replays of a graph of BLOCK launches on the rotating weight sets.
    x1 = torch.randn((1, H), device=dev).to(torch.float16)
    acts = torch.empty((1, I), dtype=torch.float16, device=dev)

    def run_gate_up():
        for r in range(BLOCK):
            layers[r % args.sets].gate_up(x1, acts)

    g_gu = graph_of(torch, run_gate_up)
    time_graph(torch, g_gu, 1, 0.3, 2)
    gu_sec = event_time_graph(torch, g_gu, 40) / BLOCK
    gu_bytes = 2 * (H * I // 2 + (H * I // G) * 3) + H * 2 + I * 2
    gu_alone = {"kernel": "gemv_kernel<F16, 1, 128, 2, true, 256, 4, 0> (hm_ffn_gate_up, whole pairs)", "avg_launch_us": round(gu_sec * 1e6, 3),
                "GB_s": round(gu_bytes / gu_sec / 1e9, 1), "frac_hbm": round(gu_bytes / gu_sec / 1e9 / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic(DECODE_TRAFFIC, "traffic_bytes_per_launch"), "algorithmic_bytes_per_launch": gu_bytes}
    log(f"gate_up GEMV alone: {gu_sec * 1e6:.2f} us, {gu_bytes / gu_sec / 1e9:.1f} GB/s")
    if args.profile == "gate_up":
        print(json.dumps({"gate_up_gemv_alone": gu_alone}), flush=True)
        return

    extra = {"decode_M1_event_median_us": round(med * 1e6, 3), "gate_up_gemv_alone": gu_alone}
    # The same layer called eagerly, one C call per layer (no graph), and the reference-signature operator's host cost.
    eg, eh = eager_bench(hm, torch, dev, layers, H, I)
    extra["decode_M1_eager"] = {"us_per_layer": round(eg, 2), "host_us_per_call": round(eh, 2), "graph_event_median_us": round(med * 1e6, 2),
                                "path": "hm_ffn_forward via ctypes, one call per layer on the rotating sets, HIP events around the enqueues"}
    if not args.quick:
        extra["decode_M1_eager"]["shim_gpuffnmodel_forward_host_us_per_call"] = round(shim_eager_host_us(hm, torch, dev, H, I), 2)
    log(f"eager decode M=1: {extra['decode_M1_eager']}")
    if not args.quick:
        for m in (4, 16):
            s, md, _, _ = decode_bench(hm, torch, dev, layers, m, H, args.steps, args.warmup, blocks=20)
            b = ffn_bytes(m, H, I, G)
            extra[f"decode_M{m}"] = {"us_per_layer": round(s * 1e6, 2), "event_median_us": round(md * 1e6, 2), "GB_s": round(b / s / 1e9, 1),
                                     "frac_hbm": round(b / s / 1e9 / HBM_PEAK_GBS, 4)}
            log(f"decode M={m}: {s * 1e6:.2f} us, {b / s / 1e9:.1f} GB/s")
        for m in (512, 2048):
            s = prefill_bench(hm, torch, dev, layers, m, H, max(6, args.steps // 24), 2)
            f = ffn_flops(m, H, I)
            extra[f"prefill_M{m}"] = {"ms_per_layer": round(s * 1e3, 3), "TFLOP_s": round(f / s / 1e12, 1),
                                       "frac_mfma": round(f / s / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
            log(f"prefill M={m}: {s * 1e3:.3f} ms, {f / s / 1e12:.1f} TFLOP/s")
        out["roofline_prefill"] = prefill_gate_up_roofline(hm, torch, dev, layers, 2048, H, I, 10)
        log(f"prefill gate_up GEMM M=2048: {out['roofline_prefill']}")
    del layers, g1, g_gu, keep
    torch.cuda.empty_cache()

    if not args.quick:
        # bf16 activations and scales (the reference operator's type): the same decode and prefill workloads.
        bl = make_layers(hm, torch, dev, H, I, G, args.sets, dtype=torch.bfloat16, seed=7)
        # 2 s of decode replays first, as for the headline: the prefill runs before leave the part in another power state
        s1, m1, _, _ = decode_bench(hm, torch, dev, bl, 1, H, args.steps, args.warmup, warm_seconds=2.0, blocks=20)
        s2 = prefill_bench(hm, torch, dev, bl, 2048, H, max(4, args.steps // 24), 2)
        b1, f2 = ffn_bytes(1, H, I, G), ffn_flops(2048, H, I)
        extra["bf16_activations"] = {"decode_M1_us": round(s1 * 1e6, 2), "decode_M1_GB_s": round(b1 / s1 / 1e9, 1),
                                     "decode_M1_event_median_us": round(m1 * 1e6, 3),
                                     "prefill_M2048_TFLOP_s": round(f2 / s2 / 1e12, 1),
                                     "prefill_M2048_frac_mfma": round(f2 / s2 / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
        log(f"bf16: {extra['bf16_activations']}")
        del bl
        torch.cuda.empty_cache()

        # 32 distinct layers, RMSNorm (eps 1e-5) + residual between layers, decode M = 1.
        stack = make_layers(hm, torch, dev, H, I, G, 32, seed=1)
        # Each layer is one pre-norm FFN block, x += FFN(RMSNorm(x) * w): two launches per layer (the norm runs in
        # the gate_up GEMV's staging, the residual add in the down GEMV's epilogue). Every token starts from its
        # embedding (a copy into x at the start of the graph), as a decoder's tokens do.
        x0 = torch.randn((1, H), device=dev).to(torch.float16)
        x = torch.empty_like(x0)
        gen = torch.Generator(device=dev)
        gen.manual_seed(11)
        norm_w = [(torch.rand(H, device=dev, generator=gen) + 0.5).to(torch.float16) for _ in stack]
        bws = torch.empty(stack[0].block_workspace_bytes(1) + 256, dtype=torch.uint8, device=dev)

        def token():
            x.copy_(x0)
            for L, w in zip(stack, norm_w):
                L.block_forward(x, w, 1e-5, workspace=bws)

        gt = graph_of(torch, token)
        time_graph(torch, gt, 1, 2.0, 4)  # 2 s of decode replays, as for the headline (the prefill runs come before)
        tok = event_time_graph(torch, gt, 128)
        assert bool(torch.isfinite(x).all()), "stack output is not finite"
        sb = 32 * ffn_bytes(1, H, I, G)
        extra["stack32_decode"] = {"us_per_token": round(tok * 1e6, 1), "ms_per_128_tokens": round(128 * tok * 1e3, 2),
                                   "GB_s": round(sb / tok / 1e9, 1), "frac_hbm": round(sb / tok / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"32-layer stack: {tok * 1e6:.1f} us/token")
        del stack, gt
        torch.cuda.empty_cache()

        # Attention Q/K/V projections through the same operator (Llama-3-8B: 4096 -> 4096 + 1024 + 1024): three
        # launches against one launch on the concatenated matrix. 24 weight sets (300 MB) rotate at M = 1 and 2048.
        extra["attention_qkv"] = qkv_bench(hm, torch, dev, H, G)
        log(f"attention QKV: {extra['attention_qkv']}")
        # The down projection kept as a pre-saved K-split pair (split at I / 2, both shares on the GPU) against
        # one matrix. 12 weight sets of each (700 MB) rotate at M = 1, 8 (470 MB) at M = 2048.
        extra["down_k_split_pair"] = ksplit_bench(hm, torch, dev, H, I, G)
        torch.cuda.empty_cache()
        log(f"down projection as a K-split pair: {extra['down_k_split_pair']}")

        # Qwen2.5-14B FFN shape, group 64.
        qh, qi, qg = 5120, 13824, 64
        ql = make_layers(hm, torch, dev, qh, qi, qg, 8, seed=2)
        s, md, _, _ = decode_bench(hm, torch, dev, ql, 1, qh, args.steps, args.warmup, warm_seconds=2.0, blocks=20)
        b = ffn_bytes(1, qh, qi, qg)
        extra["qwen14b_g64_decode_M1"] = {"us_per_layer": round(s * 1e6, 2), "event_median_us": round(md * 1e6, 3),
                                          "GB_s": round(b / s / 1e9, 1), "frac_hbm": round(b / s / 1e9 / HBM_PEAK_GBS, 4)}
        s = prefill_bench(hm, torch, dev, ql, 1024, qh, max(4, args.steps // 24), 2)
        f = ffn_flops(1024, qh, qi)
        extra["qwen14b_g64_prefill_M1024"] = {"ms_per_layer": round(s * 1e3, 3), "TFLOP_s": round(f / s / 1e12, 1),
                                               "frac_mfma": round(f / s / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
        log(f"qwen decode {extra['qwen14b_g64_decode_M1']}, prefill {extra['qwen14b_g64_prefill_M1024']}")
        del ql
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        log("CPU baseline ...")
        cpu = cpu_baseline(args.cpu_seconds, H, I, "Llama-3-8B")
        log(f"CPU: {cpu['value']} GB/s with {cpu['cores']} threads")
        c1 = cpu_baseline(min(6.0, args.cpu_seconds / 2), 2048, 8192, "Llama-3.2-1B")
        cpu["config1_llama32_1b"] = {"GB_s": c1["value"], "threads": c1["cores"], "ms_per_call": c1["ms_per_call"]}

    line = {
        "metric": "W4A16 FFN decode GB/s (%HBM peak) + prefill TFLOP/s, Llama-3-8B FFN shape",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded random W4A16 weights, N(0,1) activations)",
        "config": {"workload": "Llama-3-8B SwiGLU FFN layer decode, M=1, H=4096, I=14336, W4A16 group 128, fp16 activations",
                   "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4), "weight_sets_rotated": args.sets,
                   "bytes_per_step": nbytes,
                   "timing": "exactly `steps` layer passes enqueued as eager C ABI calls (hm_ffn_forward), wall clock with "
                             "synchronize on both sides, after untimed warm-up passes; the event median over graphs of 48 "
                             "passes is in extra"},
        "roofline": out["roofline"],
        "roofline_prefill": out.get("roofline_prefill"),
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
