"""Benchmark of the low-bit GEMM hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

A step is one launch of the 1-bit sign-weight GEMM on BASELINE.json's configs[0] workload, at the M = 128 row count
the metric quotes: A = int8 [128, 1024] per-token quantized from fp16 N(0,1) with fp16 scales, W = uniform random bits
[4096, 1024] (export codes -> native layout), fp16 per-channel scales U(0.01, 0.1), fp16 output [128, 4096] (the
int32 accumulators are written only by the parity tests, not in the timed step). Inputs are resident in HBM before
timing. Launches go through the product C ABI (a kea_lowbit_gemm plan, validated once) on one stream; to keep the host
out of the measurement the K launches are queued behind a bounded spin kernel (kea_probe_spin) that outlasts their
submission, so the GPU runs them back to back between the two HIP events (`timing.graph_us_per_step`: the same K
launches replayed as one HIP graph).

The headline is HOT: back-to-back launches on the same 640 KB of operands, which stay in the 256 MB last-level cache
between launches. `cold` repeats the measurement with every launch reading its own copy of the operands, cycling
through more than 768 MiB (three times that cache).

Prints one JSON line: value = int8 TOPS (2*M*N*K ops per step), `roofline` for the GEMM kernel (achieved = algorithmic
ops per launch / average launch time from HIP events on the launch stream), `floors` = the launch floors of the same
grid (an empty kernel, and kernels that only load the tiles' operand bytes and/or store the output), `encoder` = the
metric's second part, ms per 10-s clip of the 24-layer synthetic encoder at batch 1 and 8 with
the batch-1 error against the FP32 dense twin, and `cpu_baseline` = the oracle's C port of the reference's b1_fallback
arithmetic (unpack -> exact int32 dot -> FP32 epilogue -> fp16) on this host's cores and on one core, beside a PyTorch
CPU restatement of the reference's own oracle formula; that leg also checks the GPU output bitwise against the oracle
(`parity`), and `suite` = BASELINE.json configs 2-4 at full size (config 2 per-channel and group-128, config 3's six
encoder linears at M = 1000, config 4's single-token shapes at both weight widths, hot and cold), each with us per
launch, TOPS, GB/s and the fraction of the binding published peak. Other modes: --suite (configs 2-4 and the
reference's tuned shapes, one line each), --case (one GEMM shape), --encoder (config 5 with accuracy against the FP32
dense twin), --copy-calibration (a plain copy for the PMC traffic calibration), --sweep (every tile of the library at
the chooser's shapes), --trace-summary (a rocprofv3 kernel trace of this benchmark read the way it times).
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "kea-kernels_amd"))
sys.path.insert(0, str(ROOT))

import kea_probes  # noqa: E402  (the benchmark's probe library, include/kea_probe.h; loaded on first use)

M, N, K = 128, 4096, 1024
OPS = 2 * M * N * K
# algorithmic HBM bytes per launch: A + W (1 bit) + alpha (fp16) + per-token scales (fp16) + Y (fp16)
BYTES = M * K + N * K // 8 + 2 * N + 2 * M + 2 * M * N
PEAK_INT8_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E, 8 TB/s
METRIC = "low-bit GEMM TOPS + % int8/HBM roofline; ms per 10-s clip encoder forward"


def make_inputs(device):
    import torch
    from kea_kernels.binary import bits, kernels
    g = torch.Generator().manual_seed(1234)
    x = torch.randn(M, K, generator=g).to(torch.float16)
    s32 = x.float().abs().amax(dim=1) / 127.0
    qs = s32.to(torch.float16)                                   # fp16 per-token scales
    q = torch.clamp(torch.round(x.float() / qs.float()[:, None]), -127, 127).to(torch.int8)
    signs = torch.where(torch.rand(N, K, generator=g) < 0.5, -1, 1).to(torch.int8)
    codes = bits.pack_signs(signs)                               # the export layout
    alpha = (torch.rand(N, generator=g) * 0.09 + 0.01).to(torch.float16)
    words = kernels.relayout_codes(codes, K, 1)
    host = dict(q=q, qs=qs, codes=codes, alpha=alpha)
    dev = dict(q=q.view(1, M, K).to(device), qs=qs.view(1, M).to(device), words=words.to(device),
               alpha=alpha.to(device), y=torch.empty(M, N, dtype=torch.float16, device=device))
    return host, dev


SPIN_NS = 200_000  # the bounded spin in front of each timed region (longer than the graphs take to submit)


def replay_timed(stream, graphs, passes: int = 1) -> float:
    """Milliseconds of `passes` back-to-back replays of `graphs` on `stream`, between HIP events recorded on that
    stream; a bounded spin kernel runs first so the replays are queued before the start event executes."""
    import torch
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        kea_probes.check(kea_probes.lib().kea_probe_spin(SPIN_NS, stream.cuda_stream), "kea_probe_spin")
        start.record(stream)
        for _ in range(passes):
            for graph in graphs:
                graph.replay()
        end.record(stream)
        torch.cuda.synchronize()
    return start.elapsed_time(end)


def capture(stream, fn, count: int):
    import torch
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(count):
            fn(i)
    return graph


def queued_timed(stream, fn, steps: int, host_us: float) -> float:
    """Milliseconds of `steps` back-to-back calls of `fn` (each enqueueing one step on `stream`), between HIP events
    recorded on that stream. The calls are queued behind a bounded spin kernel that outlasts their submission
    (host_us per call, doubled), so the GPU runs them back to back with no host gaps and no graph boundaries."""
    import torch
    spin = int(min(100e6, SPIN_NS + 2e3 * host_us * steps))
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        kea_probes.check(kea_probes.lib().kea_probe_spin(spin, stream.cuda_stream), "kea_probe_spin")
        start.record(stream)
        for i in range(steps):
            fn(i)
        end.record(stream)
        torch.cuda.synchronize()
    return start.elapsed_time(end)


def gpu_bench(steps: int, warmup: int):
    import torch
    from kea_kernels import _hip, lowbit
    from kea_kernels.binary import configs
    device = torch.device("cuda", 0)
    _hip.require_gfx950(device)
    host, d = make_inputs(device)
    stream = torch.cuda.Stream(device)
    handle = stream.cuda_stream
    # the timed step: the product launch path with its validation done once (lowbit.GemmPlan)
    plan = lowbit.GemmPlan(1, d["q"], d["qs"], d["words"], N, K, d["alpha"], None, d["y"], None)

    def step(i=0):
        plan(handle)

    for _ in range(max(1, warmup)):
        step()
    torch.cuda.synchronize()
    # host cost per launch (no synchronization inside): sizes the spin that keeps submission out of the timing
    t0 = time.perf_counter()
    for _ in range(100):
        step()
    host_us = (time.perf_counter() - t0) / 100 * 1e6
    torch.cuda.synchronize()
    ms_per_step = queued_timed(stream, step, steps, host_us) / steps

    # the same K steps replayed as one HIP graph (a graph launch adds a fixed cost per replay)
    graph = capture(stream, step, steps)
    replay_timed(stream, [graph])
    graph_ms = replay_timed(stream, [graph]) / steps
    del graph

    # eager launch rate (host path included, synchronized at the end): through the plan and through lowbit.gemm;
    # warm-up calls first (the first call of a layout resolves it, the first launch of a kernel loads its code)
    def eager_us(fn, count=200):
        with torch.cuda.stream(stream):
            for _ in range(20):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(count):
                fn()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) / count * 1e6

    checked = eager_us(lambda: lowbit.gemm(1, d["q"], d["qs"], d["words"], N, K, d["alpha"], None, d["y"], None))
    planned = eager_us(step)
    # the drop-in operator a caller uses: Int8MmaLayer.linear at one part on config 1's weights (quantizer + GEMM,
    # two launches, output and int8 parts allocated per call), beside the cost of one empty kernel launch
    from kea_kernels.binary import layer_parts
    lay = layer_parts.LAYERS[1].prepare(host["codes"], host["alpha"].float(), None, K, device)
    xh = torch.randn(M, K, generator=torch.Generator().manual_seed(7)).to(torch.float16).to(device)
    with torch.cuda.stream(stream):
        layer_us = eager_us(lambda: lay.linear(xh, out_dtype=torch.float16))
        empty_us = eager_us(lambda: kea_probes.lib().kea_probe_spin(0, handle))
    cfg = configs.choose(M, N, K, parts=1, wbits=1)
    return {"ms_per_step": ms_per_step, "graph_ms_per_step": graph_ms, "host_us_per_launch": host_us,
            "eager_us": planned, "eager_checked_us": checked, "eager_layer_us": layer_us, "eager_empty_us": empty_us,
            "cfg": cfg, "host": host, "d": d, "stream": stream}


def cold_bench(d, stream, launches: int = 1300) -> float:
    """Microseconds per launch when no launch finds its operands in a cache: `launches` launches, each reading its
    own copy of q and the weight words, cycling through >= 768 MiB of copies (three times the last-level cache),
    queued behind a spin as the hot figure is."""
    import torch
    from kea_kernels import lowbit
    per_copy = d["q"].numel() + d["words"].numel() * 4
    copies = -(-(3 << 28) // per_copy)
    plans = [lowbit.GemmPlan(1, d["q"].clone(), d["qs"], d["words"].clone(), N, K, d["alpha"], None, d["y"], None)
             for _ in range(copies)]
    handle = stream.cuda_stream
    torch.cuda.synchronize()
    for pl in plans:  # one untimed pass
        pl(handle)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(100):
        plans[i % copies](handle)
    host_us = (time.perf_counter() - t0) / 100 * 1e6
    us = queued_timed(stream, lambda i: plans[i % copies](handle), launches, host_us) * 1000 / launches
    del plans
    torch.cuda.empty_cache()
    return us


def launch_floors(d, stream, tile_name: str, reps: int = 10, shape=(M, N, K), waves: int = 4) -> dict:
    """Per-launch microseconds of the launch-floor probes (include/kea_probe.h) on the GEMM's own grid: one
    workgroup of `waves` waves per BM x BN tile of the chosen configuration, doing nothing, only loading its tile's
    operand bytes, only storing its fp16 outputs, or both; graphs of 100 launches, timed as the GEMM is. d holds the
    shape's q (int8 [m][k]), native 1-bit words and fp16 y."""
    import ctypes
    import torch
    L = kea_probes.lib()
    m, n, k = shape
    bm, bn = (int(v) for v in tile_name.split()[0].split("x"))
    vp = ctypes.c_void_p
    y = torch.empty_like(d["y"])  # the probes' stores must not touch the GEMM's output (checked later)
    out = {"tile": f"{bm}x{bn}", "workgroups": (m // bm) * (n // bn), "waves": waves}
    for kind, name in enumerate(("empty_us", "loads_us", "stores_us", "loads_stores_us")):
        def probe(i, kind=kind):
            rc = L.kea_probe_floor_waves(kind, m, n, k, bm, bn, waves, vp(d["q"].data_ptr()),
                                         vp(d["words"].data_ptr()), vp(y.data_ptr()), n,
                                         vp(torch.cuda.current_stream().cuda_stream))
            kea_probes.check(rc, "kea_probe_floor")
        graph = capture(stream, probe, 100)
        replay_timed(stream, [graph])
        out[name] = round(replay_timed(stream, [graph], reps) * 1000 / (100 * reps), 3)
    return out


def probes() -> None:
    """--probes: what bounds the GEMMs, one JSON line per measurement.

    * mfma: the int8 MFMA loop at 1, 2, 4 and 8 waves per SIMD, on the fixed operand pattern and on random bytes (the
      GEMM's kind of data), best of 5 launches, for both int8 instruction shapes: v_mfma_i32_16x16x64_i8
      (kea_probe_mfma_i8_operands, the one the GEMMs use) and v_mfma_i32_32x32x32_i8 (kea_probe_mfma_i8_32);
    * exchange: what handing data to the last-arriving workgroup of a group costs inside one launch
      (kea_probe_exchange: writes only, + a relaxed arrival count, + an acquire-release count and the read), graphs of
      100 launches, at the group sizes an in-launch split-K (4) and a whole-grid exchange need;
    * config3_floors: the launch floors of config 3's grid (M = 1024 so the 128x128 tile divides it; N = 4096,
      K = 1024) with 4, 8 and 16 waves per workgroup, next to the GEMM on that grid with tile 11 (128x128, 8 waves)
      and tile 6 (the same compute waves and 8 producer waves, 16 in all), and on the other grids a large-M kernel
      could use (64x128, 64x256, 32x256 and 128x256 tiles at 8 or 16 waves: fewer activation re-reads against fewer
      or more workgroups);
    * config1_floors: the launch floors of config 1's shape on grids of 16x16 to 128x128 tiles and 1 to 8 waves per
      workgroup (how the cost of moving the operands depends on the grid)."""
    import ctypes
    import torch
    from kea_kernels import lowbit
    from kea_kernels.binary import bits, kernels
    from kea_kernels.binary.kernels import GemmConfig
    L = kea_probes.lib()
    dev = torch.device("cuda", 0)
    vp = ctypes.c_void_p
    stream = torch.cuda.Stream(dev)
    g = torch.Generator().manual_seed(0)

    def best_of(fn, reps=5):
        best = float("inf")
        with torch.cuda.stream(stream):
            for _ in range(reps + 1):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(stream)
                fn()
                b.record(stream)
                torch.cuda.synchronize()
                best = min(best, a.elapsed_time(b) * 1e-3)
        return best

    operands = {"pattern": None,
                "random": torch.randint(-2 ** 31, 2 ** 31 - 1, (128, 4), generator=g, dtype=torch.int64)
                .to(torch.int32).to(dev)}
    out = torch.empty(2048 * 256, dtype=torch.int32, device=dev)
    shapes = {"16x16x64": (L.kea_probe_mfma_i8_operands, L.kea_probe_mfma_i8_ops, 2000),
              "32x32x32": (L.kea_probe_mfma_i8_32, L.kea_probe_mfma_i8_32_ops, 1000)}
    for shape, (fn, ops_fn, iters) in shapes.items():
        for data, ops_t in operands.items():
            for blocks in (256, 512, 1024, 2048):
                def run(blocks=blocks, ops_t=ops_t, fn=fn, iters=iters):
                    rc = fn(blocks, iters, vp(ops_t.data_ptr() if ops_t is not None else 0), vp(out.data_ptr()),
                            vp(stream.cuda_stream))
                    kea_probes.check(rc, "kea_probe_mfma")
                t = best_of(run)
                print(json.dumps({"probe": "mfma", "shape": shape, "operands": data, "waves_per_simd": blocks // 256,
                                  "tops": round(ops_fn(blocks, iters) / t / 1e12, 1)}), flush=True)

    for wgs in (64, 256, 1024):
        for nbytes in (1024, 16384):
            words = nbytes // 16
            slots = torch.zeros(wgs * words * 4, dtype=torch.int32, device=dev)
            for group in sorted({4, wgs}):
                counters = torch.zeros(-(-wgs // group), dtype=torch.int32, device=dev)
                result = torch.zeros(1, dtype=torch.int32, device=dev)
                row = {"probe": "exchange", "workgroups": wgs, "bytes_per_workgroup": nbytes, "group": group}
                for kind, name in enumerate(("write_us", "count_us", "fenced_us")):
                    def launch(i=0, kind=kind):
                        rc = L.kea_probe_exchange(kind, wgs, words, group, vp(slots.data_ptr()),
                                                  vp(counters.data_ptr()), vp(result.data_ptr()),
                                                  vp(torch.cuda.current_stream().cuda_stream))
                        kea_probes.check(rc, "kea_probe_exchange")
                    graph = capture(stream, launch, 100)
                    replay_timed(stream, [graph])
                    row[name] = round(replay_timed(stream, [graph], 5) * 1000 / 500, 3)
                with torch.cuda.stream(stream):
                    result.zero_()
                    launch(kind=2)
                torch.cuda.synchronize()
                row["fenced_sum_ok"] = (int(result.item()) & 0xFFFFFFFF) == (wgs * (wgs - 1) // 2) & 0xFFFFFFFF
                print(json.dumps(row), flush=True)

    m, n, k = 1024, 4096, 1024
    q = torch.randint(-127, 128, (1, m, k), generator=g, dtype=torch.int8).to(dev)
    qs = (torch.rand(1, m, generator=g) * 0.01 + 1e-3).half().to(dev)
    codes = bits.pack_signs(torch.where(torch.rand(n, k, generator=g) < 0.5, -1, 1).to(torch.int8))
    words = kernels.relayout_codes(codes, k, 1).to(dev)
    alpha = (torch.rand(n, generator=g) * 0.09 + 0.01).half().to(dev)
    y = torch.empty(m, n, dtype=torch.float16, device=dev)
    gemm_us = {}
    for tile in (11, 6):
        gemm = capture(stream, lambda i, tile=tile: lowbit.gemm(1, q, qs, words, n, k, alpha, None, y, None,
                                                                config=GemmConfig(tile, 1)), 100)
        replay_timed(stream, [gemm])
        gemm_us[tile] = round(replay_timed(stream, [gemm], 10) * 1000 / 1000, 3)
    for tile, waves in (("128x128", 4), ("128x128", 8), ("128x128", 16), ("64x128", 8), ("64x128", 16),
                        ("64x256", 8), ("64x256", 16), ("32x256", 8), ("32x256", 16), ("128x256", 16)):
        row = {"probe": "config3_floors", "M": m, "N": n, "K": k}
        row.update(launch_floors({"q": q, "words": words, "y": y}, stream, tile, shape=(m, n, k), waves=waves))
        row["gemm_tile11_us"], row["gemm_tile6_us"] = gemm_us[11], gemm_us[6]
        print(json.dumps(row), flush=True)

    host, d = make_inputs(dev)
    for tile, waves in (("16x16", 4), ("16x32", 4), ("16x64", 1), ("16x64", 2), ("16x64", 4), ("16x64", 8),
                        ("16x128", 4), ("16x128", 8), ("32x128", 4), ("64x128", 4), ("128x128", 8)):
        row = {"probe": "config1_floors", "M": M, "N": N, "K": K}
        row.update(launch_floors(d, stream, tile, waves=waves))
        print(json.dumps(row), flush=True)


def measured_peaks(reps: int = 5) -> dict:
    """What this GPU sustains, for fractions against measured rather than published peaks: the dense int8 MFMA loop
    of the library's probe (2048 workgroups of four waves, 8 independent 16x16x64 MFMA chains each) on its fixed
    operand pattern and on random operand bytes (the kind of data a GEMM multiplies; the matrix cores sustain less on
    it), and a 1 GiB device-to-device copy (read + write bytes). Best of `reps` event-timed launches each."""
    import ctypes
    import torch
    L = kea_probes.lib()
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    blocks, iters = 2048, 2000
    out = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    ops = L.kea_probe_mfma_i8_ops(blocks, iters)
    g = torch.Generator().manual_seed(0)
    random_words = torch.randint(-2 ** 31, 2 ** 31 - 1, (128, 4), generator=g, dtype=torch.int64).to(torch.int32).to(dev)

    def timed(fn):
        best = float("inf")
        for _ in range(reps + 1):  # the first launch warms up
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            fn()
            b.record(stream)
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b) * 1e-3)
        return best

    def mfma(operands):
        rc = L.kea_probe_mfma_i8_operands(blocks, iters, ctypes.c_void_p(operands), ctypes.c_void_p(out.data_ptr()),
                                          ctypes.c_void_p(stream.cuda_stream))
        kea_probes.check(rc, "kea_probe_mfma_i8_operands")

    t_pattern = timed(lambda: mfma(None))
    t_random = timed(lambda: mfma(random_words.data_ptr()))
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    t_copy = timed(lambda: dst.copy_(src))
    nbytes = 2 * src.numel() * 4
    del src, dst
    return {"mfma_i8_tops": round(ops / t_pattern / 1e12, 1), "mfma_i8_tops_random": round(ops / t_random / 1e12, 1),
            "copy_gbs": round(nbytes / t_copy / 1e9, 1),
            "method": "int8 MFMA loop (2048 WGs x 4 waves x 2000 x 8 v_mfma_i32_16x16x64_i8) on the probe's fixed "
                      "operand pattern and on random operand bytes, and a 1 GiB device-to-device copy (read + write "
                      "bytes), best of 5; frac_of_measured uses the random-operand rate"}


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(host, y_gpu, seconds: float = 10.0) -> dict:
    """The oracle's C port of b1_fallback on the same workload, repeated for about `seconds` on this host's cores,
    then for a third of that on one core; beside it, a PyTorch CPU restatement of the reference's own oracle formula
    (q.to(int64) @ signs.to(int64).T, tests/test_kernels_gpu.py:23-27, then the FP32 epilogue) for a third of that.
    The oracle's fp16 output is also the checker of the GPU's: `parity` is "bitwise" or the count of differing
    outputs."""
    import numpy as np
    import torch
    from oracle import oracle as O
    cores = len(os.sched_getaffinity(0))
    threads = O.set_threads(min(cores, int(os.environ.get("OMP_NUM_THREADS", cores))))
    q = host["q"].numpy().reshape(1, M, K)
    codes = host["codes"].numpy()
    qs = host["qs"].float().numpy().reshape(1, M)
    alpha = host["alpha"].float().numpy()

    def timed_oracle(budget):
        reps, t0 = 0, time.perf_counter()
        while True:
            y = O.to_f16_bits(O.epilogue(O.b1_gemm(q, codes, K), qs, alpha))
            reps += 1
            if time.perf_counter() - t0 >= budget:
                return y, reps, time.perf_counter() - t0

    y, reps, elapsed = timed_oracle(seconds)
    got = y_gpu.view(torch.int16).cpu().numpy().view(np.uint16).reshape(M, N)
    mismatches = int((got != y.reshape(M, N)).sum())
    O.set_threads(1)
    _, reps1, elapsed1 = timed_oracle(seconds / 3)
    O.set_threads(threads)

    # the reference's oracle formula on PyTorch's CPU backend (int64 matmul), then the same FP32 epilogue
    signs = torch.from_numpy(O.unpack_signs(codes, K).astype(np.int8))
    q64, s64 = host["q"].to(torch.int64), signs.to(torch.int64)
    qs32, al32 = host["qs"].float(), host["alpha"].float()
    treps, t0 = 0, time.perf_counter()
    while True:
        acc = q64 @ s64.T
        yt = ((acc.to(torch.float32) * qs32[:, None]) * al32[None, :]).to(torch.float16)
        treps += 1
        if time.perf_counter() - t0 >= seconds / 3:
            break
    telapsed = time.perf_counter() - t0
    del yt
    return {"value": round(OPS * reps / elapsed / 1e12, 6), "unit": "TOPS", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{reps} full config-1 GEMMs (M=128, N=4096, K=1024, unpack + exact int32 dot + FP32 epilogue "
                      f"+ fp16 rounding) in {elapsed:.1f} s, OpenMP over output columns on {threads} threads",
            "one_core": {"value": round(OPS * reps1 / elapsed1 / 1e12, 6), "unit": "TOPS", "cores": 1,
                         "sample": f"{reps1} GEMMs in {elapsed1:.1f} s"},
            "torch_int64": {"value": round(OPS * treps / telapsed / 1e12, 6), "unit": "TOPS",
                            "cores": torch.get_num_threads(),
                            "sample": f"{treps} x (q.to(int64) @ signs.to(int64).T + FP32 epilogue + fp16) in "
                                      f"{telapsed:.1f} s, torch CPU"},
            "parity": "bitwise" if mismatches == 0 else f"{mismatches} of {M * N} fp16 outputs differ"}


TRAFFIC_PROFILE = ROOT / "profiles" / "b1_gemm_config1_traffic.json"


def kernel_sources_sha() -> str:
    """SHA-256 (16 hex digits) of the library's kernel sources (csrc/*), the build a traffic profile belongs to."""
    h = hashlib.sha256()
    for path in sorted((ROOT / "kea-kernels_amd" / "csrc").iterdir()):
        if path.suffix in (".hip", ".h", ".cpp"):
            h.update(path.name.encode())
            h.update(path.read_bytes())
    return h.hexdigest()[:16]


def traffic_from_profiles():
    """HBM bytes per launch from the committed rocprofv3 PMC summary and the kernel-source hash it was measured on,
    or (None, None) if there is none."""
    if not TRAFFIC_PROFILE.is_file():
        return None, None
    try:
        data = json.loads(TRAFFIC_PROFILE.read_text())
    except (OSError, ValueError):
        return None, None
    return data.get("hbm_bytes_per_launch"), data.get("kernel_sources_sha")


# --- secondary measurements (python bench.py --suite): BASELINE.json configs 2-4 and the reference's tuned shapes ---
REF_SHAPES = [(n, k, m) for n, k in [(1024, 1024), (1024, 4096), (2048, 1024), (3072, 1024), (4096, 1024)]
              for m in (38, 126, 256, 368)]  # kk/binary/configs.py:17-36 (RTX 5090 timings, three parts, FP32 out)


def _suite_case(wbits, parts, m, n, k, *, scale_dtype, out_dtype, seed, reps=200, ws_group=0, cold=False,
                config=None):
    """Per-launch microseconds of the library's default configuration, inputs resident, HIP-graph replay.

    cold: every launch reads its own copy of the weights and activations, cycling through at least 768 MiB of
    copies (three times the 256 MB last-level cache), so no launch finds its operands in a cache."""
    import torch
    from kea_kernels import formats, lowbit
    from kea_kernels.binary import bits, kernels
    g = torch.Generator().manual_seed(seed)
    dev = torch.device("cuda", 0)
    ldq = -(-k // 16) * 16
    q = torch.randint(-127, 128, (parts, m, ldq), generator=g, dtype=torch.int8).to(dev)
    qs = (torch.rand(parts, m, generator=g) * 0.01 + 1e-3).to(scale_dtype).to(dev)
    if wbits == 1:
        codes = bits.pack_signs(torch.where(torch.rand(n, k, generator=g) < 0.5, -1, 1).to(torch.int8))
    else:
        codes = formats.pack_ternary(torch.randint(-1, 2, (n, k), generator=g, dtype=torch.int8))
    words = kernels.relayout_codes(codes, k, wbits).to(dev)
    groups = -(-k // ws_group) if ws_group else 0
    shape = (n, groups) if ws_group else (n,)
    alpha = (torch.rand(*shape, generator=g) * 0.09 + 0.01).to(scale_dtype).to(dev)
    y = torch.empty(m, n, dtype=out_dtype, device=dev)
    stream = torch.cuda.Stream(dev)
    copies = 1
    if cold:
        per_copy = words.numel() * words.element_size() + q.numel()
        copies = -(-(3 << 28) // per_copy)
        operands = [(q.clone(), words.clone()) for _ in range(copies)]
    else:
        operands = [(q, words)]

    def step(i=0):
        qi, wi = operands[i % copies]
        lowbit.gemm(wbits, qi, qs, wi, n, k, alpha, None, y, None, ws_group=ws_group, config=config)

    with torch.cuda.stream(stream):
        step()
    torch.cuda.synchronize()
    graphs = [capture(stream, lambda i, g0=g0: step(g0 + i), 100) for g0 in range(0, max(copies, 100), 100)]
    passes = max(1, reps // (100 * len(graphs)))
    replay_timed(stream, graphs)  # one untimed pass
    us = replay_timed(stream, graphs, passes) * 1000 / (passes * 100 * len(graphs))
    del operands
    esz = {torch.float32: 4, torch.float16: 2, torch.bfloat16: 2}
    ops = 2 * m * n * k * parts
    nbytes = (m * k * parts + n * (-(-k * wbits // 8)) + esz[scale_dtype] * (alpha.numel() + parts * m)
              + esz[out_dtype] * m * n)
    t_roof = max(ops / (PEAK_INT8_TOPS * 1e12), nbytes / (PEAK_HBM_GBS * 1e9))
    return {"wbits": wbits, "parts": parts, "M": m, "N": n, "K": k, "ws_group": ws_group, "cold": cold,
            "us": round(us, 3),
            "tops": round(ops / us / 1e6, 2), "gbs": round(nbytes / us / 1e3, 1),
            "bound": "mfma" if ops / (PEAK_INT8_TOPS * 1e12) >= nbytes / (PEAK_HBM_GBS * 1e9) else "hbm",
            "roofline_frac": round(t_roof / (us * 1e-6), 4)}


# BASELINE.json configs 2-4 as named cases: (name, weight bits, M, N, K, ws_group, cold); fp16 scales and output
CONFIG3_SHAPES = [("qkv", 3072, 1024), ("attn_out", 1024, 1024), ("ffn_up", 4096, 1024), ("ffn_down", 1024, 4096),
                  ("pw1", 2048, 1024), ("pw2", 1024, 1024)]
BASELINE_CASES = ([("config2", 2, 128, 1024, 4096, 0, False), ("config2_group128", 2, 128, 1024, 4096, 128, False)]
                  + [(f"config3_{name}", 1, 1000, n, k, 0, False) for name, n, k in CONFIG3_SHAPES]
                  + [(f"config4_w{w}_{tag}_m{m}", w, m, n, k, 0, cold)
                     for cold in (False, True) for w in (1, 2) for m in (1, 4, 16)
                     for tag, n, k in [("pred", 2560, 640), ("joint", 1030, 640)]]
                  + [(f"config4_w{w}_down_m16", w, 16, 1024, 4096, 0, cold) for cold in (False, True) for w in (1, 2)])


def _case_name(name: str, cold: bool) -> str:
    return name + ("_cold" if cold else "")


def baseline_suite(reps: int = 200) -> dict:
    """BASELINE.json configs 2-4 at their full sizes, library-chosen configuration, inputs resident in HBM, HIP-graph
    replay: {case: {us, tops, gbs, bound, frac}} (frac against the binding published peak: 5.0 POP/s int8 or
    8 TB/s HBM). `_cold` cases read every launch's weights and activations from their own copy (>= 768 MiB cycled)."""
    import torch
    out = {}
    for i, (name, w, m, n, k, group, cold) in enumerate(BASELINE_CASES):
        row = _suite_case(w, 1, m, n, k, scale_dtype=torch.float16, out_dtype=torch.float16, seed=100 + i,
                          ws_group=group, cold=cold, reps=reps)
        out[_case_name(name, cold)] = {"us": row["us"], "tops": row["tops"], "gbs": row["gbs"],
                                       "bound": row["bound"], "frac": row["roofline_frac"]}
    return out


def suite() -> None:
    """One JSON line per case: configs 2-4 of BASELINE.json and the reference's tuned (N, K, M) shapes at three
    activation parts with FP32 scales and output (the arithmetic its in-source timings use)."""
    import torch
    f16, f32 = torch.float16, torch.float32
    for i, (name, w, m, n, k, group, cold) in enumerate(BASELINE_CASES):
        row = _suite_case(w, 1, m, n, k, scale_dtype=f16, out_dtype=f16, seed=100 + i, ws_group=group, cold=cold)
        print(json.dumps({"case": _case_name(name, cold), **row}), flush=True)
    cases = [("refshape_x3", w, 3, m, n, k, f32, f32) for w in (1, 2) for n, k, m in REF_SHAPES]
    for i, (name, w, p, m, n, k, sd, od) in enumerate(cases):
        row = _suite_case(w, p, m, n, k, scale_dtype=sd, out_dtype=od, seed=i)
        print(json.dumps({"case": name, **row}), flush=True)


# the chooser's shapes: BASELINE configs 1-4 and the encoder's linears (N, K) at M from single tokens to batch 8 of
# 125 frames, the reference's tuned M points among them (kk/binary/configs.py:17-36)
SWEEP_SHAPES = [(4096, 1024), (1024, 4096), (3072, 1024), (1024, 1024), (2048, 1024), (2560, 640), (1030, 640)]
SWEEP_M = (1, 16, 38, 64, 126, 256, 368, 512, 1000)


def sweep(parts_list=(1, 2, 3), wbits_list=(1, 2)) -> None:
    """One JSON line per (wbits, parts, M, N, K): per-launch microseconds of every tile configuration of the library
    (split 0: the library's split for that tile; fp16 scales and output, HIP-graph replay of 100 launches behind a
    spin) and the tile the chooser picks. The chooser table (csrc/kea_gemm_table.h) is read from these lines."""
    import torch
    from kea_kernels import formats, lowbit
    from kea_kernels.binary import bits, configs, kernels
    dev = torch.device("cuda", 0)
    stream = torch.cuda.Stream(dev)
    ntiles = kernels.tile_count()
    for wbits in wbits_list:
        for n, k in SWEEP_SHAPES:
            g = torch.Generator().manual_seed(n + k + wbits)
            if wbits == 1:
                codes = bits.pack_signs(torch.where(torch.rand(n, k, generator=g) < 0.5, -1, 1).to(torch.int8))
            else:
                codes = formats.pack_ternary(torch.randint(-1, 2, (n, k), generator=g, dtype=torch.int8))
            words = kernels.relayout_codes(codes, k, wbits).to(dev)
            alpha = (torch.rand(n, generator=g) * 0.09 + 0.01).half().to(dev)
            for parts in parts_list:
                for m in SWEEP_M:
                    ldq = -(-k // 16) * 16
                    q = torch.randint(-127, 128, (parts, m, ldq), generator=g, dtype=torch.int8).to(dev)
                    qs = (torch.rand(parts, m, generator=g) * 0.01 + 1e-3).half().to(dev)
                    y = torch.empty(m, n, dtype=torch.float16, device=dev)
                    row = {"wbits": wbits, "parts": parts, "M": m, "N": n, "K": k,
                           "chosen": configs.choose(m, n, k, parts, wbits).tile}
                    for tile in range(1, ntiles + 1):
                        try:
                            plan = lowbit.GemmPlan(wbits, q, qs, words, n, k, alpha, None, y, None,
                                                   config=kernels.GemmConfig(tile, 0))
                        except ValueError:
                            continue  # the tile does not fit this part count / K
                        graph = capture(stream, lambda i: plan(), 100)
                        replay_timed(stream, [graph])
                        row[f"t{tile}"] = round(replay_timed(stream, [graph], 3) * 1000 / 300, 3)
                        del graph, plan
                    print(json.dumps(row), flush=True)


def encoder_bench(batch: int, parts: int, reps: int = 20, seed: int = 5, check_dense: bool = True) -> dict:
    """the 24-layer synthetic encoder (1-bit linears at `parts` int8 parts) on `batch` clips
    of 10 s of seeded Gaussian noise, preprocessing + encoder captured in one HIP graph; ms per clip = replay / batch.
    Accuracy: relative Frobenius error against the same model with FP32 dense linears."""
    import torch
    from kea_kernels import encoder as E
    cfg = E.EncoderConfig()
    weights = E.synthetic_weights(cfg, seed=seed)
    enc = E.FastConformerEncoder(weights, cfg, "cuda", parts=parts)
    g = torch.Generator().manual_seed(seed + batch)
    audio = torch.randn(batch, 160000, generator=g).cuda()
    t0 = time.perf_counter()
    enc(audio)
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3
    out = enc(audio)  # a second eager call: library autotuning (convolutions, FFT plans) settled
    graph = E.EncoderGraph(enc, batch, 160000)
    got = graph(audio).clone()
    torch.cuda.synchronize()
    graph_diff = float((got - out).abs().max())
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(graph.stream):  # replays back to back on the graph's own stream
        for _ in range(3):
            graph.graph.replay()
        a.record(graph.stream)
        for _ in range(reps):
            graph.graph.replay()
        b.record(graph.stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    rel = None
    if check_dense:
        dense = E.FastConformerEncoder(weights, cfg, "cuda", dense=True)
        ref = dense(audio)
        rel = float((out.double() - ref.double()).norm() / ref.double().norm())
        del dense, ref
    t = out.shape[1]
    # linear ops per forward: the 10 per-token linears of each layer (W_pos runs once per length, outside the graph)
    per_layer = sum(n * k for name, (n, k, _) in E.quantized_shapes(cfg).items() if name != "self_attn.linear_pos")
    lin_ops = 2 * t * batch * cfg.layers * per_layer
    return {"case": "config5_encoder", "batch": batch, "parts": parts, "frames": t, "ms_per_forward": round(ms, 4),
            "ms_per_clip": round(ms / batch, 4), "eager_ms_first_call": round(eager_ms, 1),
            "graph_vs_eager_max_abs_diff": graph_diff, "rel_err_vs_dense_fp32": rel,
            "quantized_linear_ops_per_clip": lin_ops // batch, "weight_bytes": enc.weight_bytes()}


def trace_summary(csv_path: str) -> dict:
    """--trace-summary: a rocprofv3 kernel trace (`<name>_kernel_trace.csv`) of this benchmark read the way the
    benchmark times: every run of back-to-back dispatches of one kernel that directly follows a bounded spin kernel
    (the queued regions of the headline figure and of the graph replays) gives (last end - first start) / dispatches,
    beside the mean and median of the traced per-dispatch durations of the same dispatches, and the median over the
    isolated ones: dispatches that start at least 1 us after the previous one ended, whose traced duration holds no
    wait behind the previous dispatch (where the profiler lets dispatches abut, their start timestamps can precede the
    previous kernel's completion processing). Nanosecond timestamps."""
    import csv
    import statistics
    with open(csv_path, newline="") as handle:
        rows = sorted(csv.DictReader(handle), key=lambda r: int(r["Start_Timestamp"]))
    regions = []
    i = 0
    while i < len(rows):
        if "spin_kernel(" in rows[i]["Kernel_Name"]:
            j = i + 1
            if j < len(rows):
                name = rows[j]["Kernel_Name"]
                k = j
                while k < len(rows) and rows[k]["Kernel_Name"] == name:
                    k += 1
                run = rows[j:k]
                durations = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in run]
                span = int(run[-1]["End_Timestamp"]) - int(run[0]["Start_Timestamp"])
                gaps = [int(b["Start_Timestamp"]) - int(a["End_Timestamp"]) for a, b in zip(run, run[1:])]
                isolated = [d for d, gap in zip(durations[1:], gaps) if gap >= 1000]
                label = name.replace("void ", "", 1).replace("(anonymous namespace)::", "")
                regions.append({"kernel": label[:label.find("(")] if "(" in label else label, "dispatches": len(run),
                                "span_us_per_dispatch": round(span / len(run) / 1e3, 4),
                                "mean_duration_us": round(statistics.fmean(durations) / 1e3, 4),
                                "median_duration_us": round(statistics.median(durations) / 1e3, 4),
                                "median_gap_us": round(statistics.median(gaps) / 1e3, 4) if gaps else None,
                                "isolated_dispatches": len(isolated),
                                "isolated_median_us": round(statistics.median(isolated) / 1e3, 4) if isolated
                                else None})
                i = k
                continue
        i += 1
    return {"trace": str(csv_path), "regions": regions}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="low-bit GEMM benchmark (BASELINE.json config 1)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-encoder", action="store_true",
                    help="skip the config-5 encoder figures (ms per 10-s clip) of the headline line")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-peaks", action="store_true",
                    help="skip the measured-peak microbenchmarks (int8 MFMA loop, 1 GiB copy)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (5 times); the known byte count "
                         "calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--encoder", action="store_true",
                    help="only run BASELINE.json config 5 (24-layer encoder, batch 1 and 8; one JSON line each)")
    ap.add_argument("--encoder-cases", default="1x1,8x1,1x3,8x3", metavar="BxP,...",
                    help="batch x parts cases of --encoder")
    ap.add_argument("--no-check-dense", action="store_true",
                    help="--encoder: skip the FP32 dense comparison (profiles then hold only the quantized encoder)")
    ap.add_argument("--suite", action="store_true",
                    help="only time BASELINE.json configs 2-4 and the reference's tuned shapes (one JSON line each)")
    ap.add_argument("--case", default=None, metavar="BITS,P,M,N,K[,TILE][;...]",
                    help="only time GEMM shapes (fp16 scales and output; the library-chosen configuration, or "
                         "tile id TILE unsplit) for --steps launches each; used for the rocprofv3 counter passes of "
                         "the larger configs")
    ap.add_argument("--ws-group", type=int, default=0, help="--case: per-group weight scales of this group size")
    ap.add_argument("--sweep", default=None, metavar="PARTS",
                    help="only time every tile configuration at the chooser's shapes for these part counts "
                         "(e.g. 1,2,3; one JSON line per shape)")
    ap.add_argument("--sweep-wbits", default="1,2", metavar="BITS",
                    help="--sweep: the weight widths to sweep (e.g. 1 or 1,2)")
    ap.add_argument("--probes", action="store_true",
                    help="only run the bounding probes: int8 MFMA rate by occupancy and operand data, the cost of a "
                         "cross-workgroup exchange inside one launch, and config 3's launch floors")
    ap.add_argument("--no-cold", action="store_true", help="skip the cold-cache config-1 figure")
    ap.add_argument("--no-floors", action="store_true", help="skip the launch-floor probes")
    ap.add_argument("--no-suite", action="store_true",
                    help="skip the `suite` object (BASELINE.json configs 2-4, library-chosen configurations)")
    ap.add_argument("--trace-summary", default=None, metavar="CSV",
                    help="only summarise a rocprofv3 kernel trace of this benchmark: per-dispatch time of every "
                         "queued region ((last end - first start) / dispatches) beside the traced mean duration")
    args = ap.parse_args(argv)
    if args.trace_summary:
        print(json.dumps(trace_summary(args.trace_summary)), flush=True)
        return 0
    if args.suite:
        suite()
        return 0
    if args.probes:
        probes()
        return 0
    if args.sweep:
        sweep(tuple(int(v) for v in args.sweep.split(",")), tuple(int(v) for v in args.sweep_wbits.split(",")))
        return 0
    if args.case:
        import torch
        from kea_kernels.binary.kernels import GemmConfig
        for spec in args.case.split(";"):
            fields = [int(v) for v in spec.split(",")]
            w, p, m, n, k = fields[:5]
            tile = fields[5] if len(fields) > 5 else 0
            try:
                row = _suite_case(w, p, m, n, k, scale_dtype=torch.float16, out_dtype=torch.float16, seed=0,
                                  reps=max(100, args.steps // 100 * 100), ws_group=args.ws_group,
                                  config=GemmConfig(tile, 1) if tile else None)
            except ValueError as e:  # a tile that does not take this shape
                row = {"error": str(e)}
            print(json.dumps({"case": "gemm", "tile": tile, **row}), flush=True)
        return 0
    if args.encoder:
        for case in args.encoder_cases.split(","):
            batch, parts = (int(v) for v in case.split("x"))
            print(json.dumps(encoder_bench(batch, parts, check_dense=not args.no_check_dense)), flush=True)
        return 0
    if args.copy_calibration:
        import torch
        src = torch.ones(args.copy_calibration << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": src.numel() * 4, "launches": 5}), flush=True)
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (data-parallel serving would "
              "shard by clip, one process per GPU). Run with --gpus 1.", file=sys.stderr)
        return 2
    if args.steps < 1:
        print("--steps must be >= 1", file=sys.stderr)
        return 2
    r = gpu_bench(args.steps, args.warmup)
    ms_per_step, cfg, host, d, stream = r["ms_per_step"], r["cfg"], r["host"], r["d"], r["stream"]
    tops = OPS / (ms_per_step * 1e-3) / 1e12
    mfma_time = OPS / (PEAK_INT8_TOPS * 1e12)
    hbm_time = BYTES / (PEAK_HBM_GBS * 1e9)
    bound = "mfma" if mfma_time >= hbm_time else "hbm"
    if bound == "mfma":
        achieved, peak, unit = tops, PEAK_INT8_TOPS, "TOPS"
    else:
        achieved, peak, unit = BYTES / (ms_per_step * 1e-3) / 1e9, PEAK_HBM_GBS, "GB/s"
    traffic, traffic_sha = traffic_from_profiles()
    line = {
        "metric": METRIC,
        "value": round(tops, 3),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "config1: 1-bit sign-weight x int8 GEMM, M=128 K=1024 N=4096, 1 activation part, "
                               "fp16 per-token and per-channel scales, fp16 output, inputs resident in HBM; HOT: "
                               "back-to-back launches on the same 640 KB of operands, which stay in the 256 MB "
                               "last-level cache (the cold figure is `cold`)",
                   "M": M, "N": N, "K": K, "parts": 1, "weight_bits": 1, "tile": cfg.label()},
        "roofline": {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
                     "frac": round(achieved / peak, 5), "traffic": traffic,
                     "traffic_build": {"kernel_sources_sha": traffic_sha,
                                       "this_build": kernel_sources_sha(),
                                       "same_build": traffic_sha == kernel_sources_sha()},
                     "algorithmic_bytes": BYTES, "ops": OPS},
        "timing": {"method": "the K launches (a validated lowbit.GemmPlan each) queued behind a bounded spin kernel "
                             "that outlasts their submission, HIP events on the launch stream around them",
                   "host_us_per_launch": round(r["host_us_per_launch"], 3),
                   "graph_us_per_step": round(r["graph_ms_per_step"] * 1e3, 3),
                   "graph_note": "the same K launches replayed as one HIP graph; a replay adds a fixed cost"},
        "eager_launch_us": round(r["eager_us"], 3),
        "eager_launch_us_checked": round(r["eager_checked_us"], 3),
        "eager_layer_us": round(r["eager_layer_us"], 3),
        "eager_empty_launch_us": round(r["eager_empty_us"], 3),
    }
    if not args.no_cold:
        cold_us = cold_bench(d, stream)
        line["cold"] = {"us_per_step": round(cold_us, 3), "tops": round(OPS / cold_us / 1e6, 3),
                        "frac": round(mfma_time / (cold_us * 1e-6), 5),
                        "method": "every launch reads its own copy of q and the weight words, cycling through "
                                  ">= 768 MiB of copies (3x the last-level cache); HIP-graph replay"}
    if not args.no_floors:
        name = _hip_config_name(cfg.tile)
        floors = launch_floors(d, stream, name, waves=_config_waves(name))
        floors["gemm_us"] = round(ms_per_step * 1e3, 3)
        line["floors"] = floors
    if not args.no_suite:
        # BASELINE.json configs 2-4 at full size (the per-shape table the reference keeps in kk/binary/configs.py)
        line["suite"] = baseline_suite()
    if not args.no_peaks:
        peaks = measured_peaks()
        measured = peaks["mfma_i8_tops_random"] if bound == "mfma" else peaks["copy_gbs"]
        line["roofline"]["measured_peak"] = measured
        line["roofline"]["frac_of_measured"] = round(achieved / measured, 5)
        line["measured_peaks"] = peaks
    if not args.no_encoder:
        # the metric's second part: ms per 10-s clip of the 24-layer encoder (config 5), one int8 part, HIP graph;
        # batch 1 also carries its error against the same model with FP32 dense linears
        enc = {f"batch{b}": encoder_bench(b, 1, check_dense=(b == 1)) for b in (1, 8)}
        line["encoder"] = {"ms_per_clip_batch1": enc["batch1"]["ms_per_clip"],
                           "ms_per_clip_batch8": enc["batch8"]["ms_per_clip"], "parts": 1,
                           "rel_err_vs_dense_fp32_batch1": enc["batch1"]["rel_err_vs_dense_fp32"],
                           "workload": "config5: 10 s of 16 kHz noise -> log-mel -> 8x subsampling -> 24 FastConformer "
                                       "layers (d 1024, 8 heads, FFN 4096, conv k 9), 1-bit linears, random init"}
    if not args.no_cpu:
        import torch
        torch.cuda.synchronize()
        line["cpu_baseline"] = cpu_baseline(host, d["y"], args.cpu_seconds)
        line["parity"] = line["cpu_baseline"]["parity"]
    print(json.dumps(line), flush=True)
    if line.get("parity", "bitwise") != "bitwise":
        print(f"bench.py: the GPU output differs from the oracle: {line['parity']}", file=sys.stderr)
        return 1
    return 0


def _hip_config_name(tile: int) -> str:
    from kea_kernels import _hip
    return _hip.lib().kea_config_name(tile).decode()


def _config_waves(name: str) -> int:
    """Waves per workgroup of a tile from its name: "16x64 k/4" (wave-split: K over 4 waves) or
    "128x128 w2x4 r4x2" (LDS ring: 2 x 4 waves)."""
    for field in name.split()[1:]:
        if field.startswith("k/"):
            return int(field[2:])
        if field.startswith("w"):
            a, b = field[1:].split("x")
            return int(a) * int(b)
    raise ValueError(f"no wave count in tile name {name!r}")


if __name__ == "__main__":
    sys.exit(main())
