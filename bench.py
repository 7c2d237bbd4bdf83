"""Benchmark of the W4A16 hot path on one MI355X ([3]).

    python bench.py [--gpus 1] [--steps 160] [--warmup 32]

A *step* is one M=1 (decode) pass over the seven linears of one
Llama-3.2-1B decoder block (q/o 2048x2048, k/v 512x2048, gate/up 8192x2048,
down 2048x8192; N x K), G=128, bf16 activations, as ONE grouped launch
(``w4a16_matmul_grouped``).  Step i uses weight set i % 16: 16 distinct
seeded sets (16 x 32.3 MB > the 256 MB Infinity Cache) so weights stream from
HBM.  Inputs are resident in HBM before the timed region.  Exactly --warmup
untimed steps run, then exactly --steps timed steps, each one call of the
library's C-ABI grouped entry point issued back to back from a C loop,
bracketed by host synchronisation and HIP events on the launch stream.

Printed (last line, JSON): ``value`` = algorithmic HBM bytes of the block
(sum N*K/2 + 4*N*K/G + 2*K + 2*N = 32,397,312 B) / time per step, in GB/s,
plus ``roofline`` for the dominant kernel (the grouped decode launch, one per
step) and ``cpu_baseline`` (the reference's torch CPU path -- dequantize to
bf16, then F.linear -- on all of this host's cores, over the same block).
Extra fields carry the per-linear (7-launch) decode block, the small-M blocks,
the M = 128/512/2048 prefill TFLOPS with a hipBLASLt bf16 reference, the
quantize kernel, HBM read ceilings and the end-to-end Llama-3.2-1B run.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "itmo-final-project_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

LINEARS = [("q_proj", 2048, 2048), ("k_proj", 512, 2048), ("v_proj", 512, 2048), ("o_proj", 2048, 2048),
           ("gate_proj", 8192, 2048), ("up_proj", 8192, 2048), ("down_proj", 2048, 8192)]
G = 128
HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, published
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, published
METRIC = "µs & HBM GB/s per 7-linear block at M=1; W4A16 TFLOPS at M=2048"


def block_bytes(M: int, g: int = G) -> int:
    return sum(N * K // 2 + 4 * N * K // g + 2 * M * K + 2 * M * N for _, N, K in LINEARS)


def lin_bytes(N: int, K: int, M: int = 1, g: int = G) -> int:
    """Algorithmic bytes of one linear: packed weights, scales + zeros, x, y."""
    return N * K // 2 + 4 * N * K // g + 2 * M * K + 2 * M * N


def block_flops(M: int) -> int:
    return sum(2 * M * N * K for _, N, K in LINEARS)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def graph_of(fn, stream, eager_warmup: bool = True):
    import torch

    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        if eager_warmup:
            fn()  # warm-up outside the graph
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=stream):
            fn()
    torch.cuda.synchronize()
    return g


def time_graph_once(g, stream) -> float:
    """ms of ONE replay, bracketed by host synchronisation, HIP events on the
    replay stream."""
    import torch

    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    host_spin(2.0)
    with torch.cuda.stream(stream):
        e0.record(stream)
        g.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def time_graph(g, reps: int, stream) -> float:
    """ms per replay, events recorded on the replay stream, bracketed by syncs."""
    import torch

    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    host_spin(2.0)
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def cpu_info() -> dict:
    """Host CPU model and the cores this process may run on (the CPU timings'
    thread count)."""
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "cores": len(os.sched_getaffinity(0))}


def _median_s(fn, reps: int) -> float:
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(sorted(ts)[len(ts) // 2])


def cpu_baseline(packed, xs, reps: int) -> dict:
    """The reference's torch CPU path on this host's cores: per linear,
    ``dequantize_int4_ref(qweight, scales, zeros, bf16)`` then
    ``F.linear(x, W_hat)`` (int4_triton/quantize.py:128-135,
    tests/test_kernels.py:56-57), restated as this package's own torch-op
    functions; ``packed``/``xs`` are the CPU copies of the M=1 block's inputs.
    Median of ``reps`` passes after one warm-up pass; also the matmul alone on
    pre-dequantized weights."""
    import torch
    import torch.nn.functional as F

    from int4_hip.quantize import dequantize_int4_ref

    info = cpu_info()
    torch.set_num_threads(info["cores"])

    def block():
        for (qw, sc, ze), x in zip(packed, xs):
            F.linear(x, dequantize_int4_ref(qw, sc, ze, torch.bfloat16))

    block()
    t = _median_s(block, reps)
    per = {}
    for (name, _, _), (qw, sc, ze), x in zip(LINEARS, packed, xs):
        per[name] = round(_median_s(lambda: F.linear(x, dequantize_int4_ref(qw, sc, ze, torch.bfloat16)), 3) * 1e3, 3)
    w_hat = [dequantize_int4_ref(qw, sc, ze, torch.bfloat16) for qw, sc, ze in packed]
    t_mm = _median_s(lambda: [F.linear(x, w) for x, w in zip(xs, w_hat)], reps)
    return {"value": round(block_bytes(1) / t / 1e9, 6), "unit": "GB/s", "cores": info["cores"],
            "threads": torch.get_num_threads(), "cpu_model": info["cpu_model"], "kind": "port", "impl": "torch",
            "sample": f"torch CPU path (dequantize_int4_ref to bf16, then F.linear) over the 7-linear block at "
                      f"M=1, G=128, one weight set, median of {reps} passes ({t * 1e3:.1f} ms per block)",
            "ms_per_block": round(t * 1e3, 3),
            "matmul_only_ms_per_block": round(t_mm * 1e3, 3),
            # the single 2048 x 2048 linear is q_proj's shape
            "per_linear_ms": per}


def cpu_numpy_port(packed_np, xs_bits, reps: int) -> dict:
    """The numpy oracle (a single-threaded restatement of the same path) over the
    same block, kept beside the torch figure."""
    import numpy as np

    from oracle import w4a16_oracle as O

    def block():
        for (qw, s, z), xb in zip(packed_np, xs_bits):
            O.w4a16_matmul(xb, "bf16", qw, s, z, accumulate="f32")

    t = _median_s(block, reps)
    return {"value": round(block_bytes(1) / t / 1e9, 6), "unit": "GB/s", "cores": 1, "kind": "port",
            "impl": "numpy", "ms_per_block": round(t * 1e3, 3),
            "sample": f"numpy oracle over the M=1 block, median of {reps} passes"}


def cpu_quantize_baseline(ws, q_bytes: int, reps: int) -> dict:
    """The reference's torch quantizer on the CPU (``quantize_int4_ref``,
    int4_triton/quantize.py:102-117, restated as this package's torch-op
    function) over the 7 block weights (bf16 CPU tensors), on all cores."""
    import torch

    from int4_hip.quantize import quantize_int4_ref

    info = cpu_info()
    torch.set_num_threads(info["cores"])

    def block():
        for w in ws:
            quantize_int4_ref(w, G)

    block()
    t = _median_s(block, reps)
    return {"value": round(q_bytes / t / 1e9, 6), "unit": "GB/s", "cores": info["cores"],
            "threads": torch.get_num_threads(), "cpu_model": info["cpu_model"], "kind": "port", "impl": "torch",
            "sample": f"torch quantize_int4_ref over the 7 block weights (G=128, bf16), "
                      f"median of {reps} passes ({t * 1e3:.1f} ms per block)",
            "ms_per_block": round(t * 1e3, 3)}


def device_copy_gbps(dev, stream, nbytes: int = 1 << 30, reps: int = 10) -> float:
    """Measured HBM rate of a plain device-to-device copy (read + write bytes
    over time), beside the 8 TB/s datasheet peak the roofline uses."""
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    with torch.cuda.stream(stream):
        for _ in range(2):
            dst.copy_(src)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            dst.copy_(src)
        e1.record(stream)
    e1.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del src, dst
    return 2 * nbytes / (ms * 1e-3) / 1e9


def hbm_read_ceiling(dev, stream, block_bytes_: int, nsets: int) -> dict | None:
    """Measured read ceilings (csrc/bench/read_probe.hip, kernels that only
    read): one long stream over 1 GiB, and the best single launch over the
    decode block's bytes -- one 1024-thread workgroup per CU, each reading a
    contiguous slice with every load in flight -- over ``nsets`` rotated
    buffers from a graph (default and non-temporal loads; also the older
    grid-stride launch of 512 workgroups)."""
    import ctypes

    import torch

    path = ROOT / "itmo-final-project_amd" / "int4_hip" / "libw4_bench.so"
    if not path.exists():
        log(f"{path} not built; no read ceiling")
        return None
    lib = ctypes.CDLL(str(path))
    fn = lib.w4bench_read
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    fs = lib.w4bench_read_slices
    fs.restype = ctypes.c_int
    fs.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    sink = torch.zeros(16, dtype=torch.int32, device=dev)
    raw = stream.cuda_stream
    cus = torch.cuda.get_device_properties(dev).multi_processor_count

    def launch(buf, nbytes, grid, block):
        rc = fn(buf.data_ptr(), nbytes, grid, block, sink.data_ptr(), raw)
        if rc != 0:
            raise RuntimeError(f"w4bench_read failed ({rc})")

    def slices(buf, nbytes, nt):
        rc = fs(buf.data_ptr(), nbytes, cus, nt, sink.data_ptr(), raw)
        if rc != 0:
            raise RuntimeError(f"w4bench_read_slices failed ({rc})")

    big = torch.ones(1 << 28, dtype=torch.int32, device=dev)  # 1 GiB
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        for _ in range(2):
            launch(big, big.numel() * 4, 2048, 256)
        e0.record(stream)
        for _ in range(10):
            launch(big, big.numel() * 4, 2048, 256)
        e1.record(stream)
    e1.synchronize()
    stream_gbps = 10 * big.numel() * 4 / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del big
    n16 = block_bytes_ // 16 * 16
    bufs = [torch.ones(n16 // 4, dtype=torch.int32, device=dev) for _ in range(nsets)]
    out = {"stream_1gib_gbps": round(stream_gbps, 1)}
    for key, body in (("slices", lambda: [slices(b, n16, 0) for b in bufs]),
                      ("slices_nt", lambda: [slices(b, n16, 1) for b in bufs]),
                      ("grid_stride", lambda: [launch(b, n16, 512, 1024) for b in bufs])):
        g = graph_of(body, stream)
        time_graph(g, 3, stream)
        us = time_graph(g, 10, stream) / nsets * 1e3
        del g
        out[f"single_launch_{key}_us"] = round(us, 3)
        out[f"single_launch_{key}_gbps"] = round(n16 / (us * 1e-6) / 1e9, 1)
    del bufs
    best = min(out["single_launch_slices_us"], out["single_launch_slices_nt_us"], out["single_launch_grid_stride_us"])
    out["single_launch_block_bytes_us"] = best
    out["single_launch_block_bytes_gbps"] = round(n16 / (best * 1e-6) / 1e9, 1)
    out["note"] = (f"read-only kernels, 16-byte loads, {n16} B per launch over {nsets} rotated buffers, graph "
                   f"replay; slices: {cus} workgroups x 1024 threads, one contiguous slice each, all loads of a "
                   "thread issued before use (default / non-temporal loads); grid_stride: 512 x 1024 threads; "
                   "stream: 2048 x 256 threads over 1 GiB")
    return out


PROFILE = ROOT / "profiles" / "dec_kernel_one_decode_block_m1.md"
ROOFLINE_KERNEL = "dec_kernel_one<0, 2, 1>"


def host_spin(ms: float) -> None:
    """Keep this host core busy for `ms` milliseconds, outside any timed
    region.  After a synchronisation that waited a while the core idles at a
    low clock, and the first ~20 library calls that follow take 6-8 us of
    host time each instead of about 3 (measured on the MI355X box), so a short
    run of steps would measure the host's wake-up instead of the GPU."""
    end = time.perf_counter() + ms * 1e-3
    while time.perf_counter() < end:
        pass


def summarize_prof(d: Path, kernel: str = ROOFLINE_KERNEL) -> str:
    """Markdown lines from a rocprofv3 run directory laid out as
    ``trace/`` (--kernel-trace --stats), ``fetch/`` (--pmc FETCH_SIZE),
    ``write/`` (--pmc WRITE_SIZE) and optionally ``sq/``, each written with
    ``--output-format csv -o run``.  FETCH_SIZE / WRITE_SIZE are scaled by what
    they read for the 32 MiB device copy of ``--copy-calib``."""
    import csv

    def rows(sub, name):
        f = d / sub / f"run_{name}.csv"
        return list(csv.DictReader(open(f))) if f.exists() else []

    def counter(sub, name, match):
        vals = [float(r["Counter_Value"]) for r in rows(sub, "counter_collection")
                if match(r["Kernel_Name"]) and r["Counter_Name"] == name]
        return sum(vals) / len(vals) if vals else None

    def first_dispatch(sub, name, match):
        # the calibration copy is the run's first device copy (later copies,
        # e.g. the 1 GiB copy-rate measurement, move other sizes)
        rs = [r for r in rows(sub, "counter_collection") if match(r["Kernel_Name"]) and r["Counter_Name"] == name]
        if not rs:
            return None
        first = min(int(r["Dispatch_Id"]) for r in rs)
        return sum(float(r["Counter_Value"]) for r in rs if int(r["Dispatch_Id"]) == first)

    out = []
    stats = [r for r in rows("trace", "kernel_stats") if kernel in r["Name"]]
    dur_ns = float(stats[0]["AverageNs"]) if stats else None
    if stats:
        r = stats[0]
        out.append(f"- kernel `{r['Name']}`: {r['Calls']} calls, average {float(r['AverageNs']) / 1e3:.3f} us, "
                   f"min {float(r['MinNs']) / 1e3:.3f} us, max {float(r['MaxNs']) / 1e3:.3f} us")
    is_copy = lambda n: "copyBuffer" in n  # noqa: E731
    is_k = lambda n: kernel in n  # noqa: E731
    f_copy, w_copy = first_dispatch("fetch", "FETCH_SIZE", is_copy), first_dispatch("write", "WRITE_SIZE", is_copy)
    f_k, w_k = counter("fetch", "FETCH_SIZE", is_k), counter("write", "WRITE_SIZE", is_k)
    traffic = None
    if None not in (f_copy, w_copy, f_k, w_k):
        fs, ws = 32768.0 / f_copy, 32768.0 / w_copy  # KiB actually moved by the 32 MiB copy
        traffic = (f_k * fs + w_k * ws) * 1024
        out.append(f"- calibration (32 MiB device copy): FETCH_SIZE {f_copy:.1f} KiB -> factor {fs:.3f}; "
                   f"WRITE_SIZE {w_copy:.1f} KiB -> factor {ws:.3f}")
        out.append(f"- per dispatch: FETCH_SIZE {f_k:.1f} KiB (x{fs:.3f} = {f_k * fs * 1024 / 1e6:.3f} MB), "
                   f"WRITE_SIZE {w_k:.1f} KiB (x{ws:.3f} = {w_k * ws * 1024 / 1e6:.3f} MB)")
        out.append(f"- traffic_bytes_per_launch: {traffic:.0f}")
        out.append(f"- algorithmic bytes per launch: {block_bytes(1)} "
                   f"(traffic / algorithmic = {traffic / block_bytes(1):.3f})")
        if dur_ns:
            out.append(f"- algorithmic rate at the traced duration: {block_bytes(1) / dur_ns:.1f} GB/s")
    sq = {}
    for r in rows("sq", "counter_collection"):
        if is_k(r["Kernel_Name"]):
            sq.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    if sq:
        out.append("- SQ counters per dispatch: " + ", ".join(
            f"{k} {sum(v) / len(v):.0f}" for k, v in sorted(sq.items())))
    return "\n".join(out)


def summarize_prefill_prof(d: Path) -> str:
    """Markdown tables of the prefill section (``--only prefill``) from a
    rocprofv3 run directory laid out as for ``summarize_prof`` (``trace/``,
    ``fetch/``, ``write/``, ``sq/``).  The section's own dispatches are matched
    to linears by their order, which every run repeats: per M, the 7-linear
    block graph (one eager pass and 13 replays), then each linear's graph of 4
    calls (13 x 4 calls), then the fused 4-call block (14 passes); a call is
    one main kernel, plus the split-K reduce where the plan splits K.  Times
    average the last 40 calls of a linear's graph (its 10 timed replays)."""
    import csv

    def ours(sub, name):
        f = d / sub / f"run_{name}.csv"
        if not f.exists():
            return []
        # the GEMM kernels only (the weight sets' quantization and the
        # dequantization for the hipBLASLt comparison are left out)
        rs = [r for r in csv.DictReader(open(f)) if "w4::" in r["Kernel_Name"] and "quantize" not in r["Kernel_Name"]]
        return sorted(rs, key=lambda r: int(r["Dispatch_Id"]))

    trace = ours("trace", "kernel_trace")
    seq = [(r["Kernel_Name"], r["Grid_Size_X"]) for r in trace]

    def counters(sub):
        # per dispatch (in order of our dispatches): {counter: value}
        byd = {}
        for r in ours(sub, "counter_collection"):
            byd.setdefault(int(r["Dispatch_Id"]), {})[r["Counter_Name"]] = float(r["Counter_Value"])
        return [byd[k] for k in sorted(byd)]

    fetch, write, sq = counters("fetch"), counters("write"), counters("sq")
    calib = {}
    for sub, cname in (("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE")):
        f = d / sub / "run_counter_collection.csv"
        if f.exists():
            rs = [r for r in csv.DictReader(open(f)) if "copyBuffer" in r["Kernel_Name"] and r["Counter_Name"] == cname]
            if rs:
                first = min(int(r["Dispatch_Id"]) for r in rs)
                calib[cname] = 32768.0 / sum(float(r["Counter_Value"]) for r in rs if int(r["Dispatch_Id"]) == first)

    def period(pos, reps, lo=1):
        for L in range(lo, (len(seq) - pos) // reps + 1):
            if seq[pos:pos + reps * L] == seq[pos:pos + L] * reps:
                return L
        raise ValueError(f"no repeating dispatch pattern at {pos}")

    def dur(i):
        return (int(trace[i]["End_Timestamp"]) - int(trace[i]["Start_Timestamp"])) / 1e3

    def avg(idx, f):
        vals = [f(i) for i in idx]
        vals = [v for v in vals if v is not None]
        return sum(vals) / len(vals) if vals else None

    def cval(rows, i, name):
        return rows[i].get(name) if i < len(rows) else None

    def short(name):
        return name.replace("void ", "").split("(")[0]

    def wgs(i):
        return int(trace[i]["Grid_Size_X"]) // max(1, int(trace[i]["Workgroup_Size_X"]))

    lines = ["| M | linear | main kernel | WGs | main us | reduce us | TFLOP/s | traffic MB | alg. MB | "
             "MFMA busy % | VALU / MFMA instr. | LDS bank conflicts |", "|---|---|---|---|---|---|---|---|---|---|---|---|"]
    fused = ["| M | call | kernel(s) | WGs | main us | reduce us | MFMA busy % |", "|---|---|---|---|---|---|---|"]
    pos = 0
    for M in (128, 512, 2048):
        pos += 14 * period(pos, 14, 7)  # the 7-linear block graph
        for name, N, K in LINEARS:
            L = period(pos, 52)
            calls = [pos + c * L for c in range(52)][-40:]
            main = calls
            red = [c + 1 for c in calls] if L == 2 else []
            t_main = avg(main, dur)
            t_red = avg(red, dur) if red else 0.0
            fs, ws = calib.get("FETCH_SIZE"), calib.get("WRITE_SIZE")
            traffic = None
            if fs and ws:
                f_kib = avg(main, lambda i: cval(fetch, i, "FETCH_SIZE")) or 0.0
                w_kib = avg(main, lambda i: cval(write, i, "WRITE_SIZE")) or 0.0
                if red:
                    f_kib += avg(red, lambda i: cval(fetch, i, "FETCH_SIZE")) or 0.0
                    w_kib += avg(red, lambda i: cval(write, i, "WRITE_SIZE")) or 0.0
                traffic = (f_kib * fs + w_kib * ws) * 1024 / 1e6
            busy = avg(main, lambda i: cval(sq, i, "SQ_VALU_MFMA_BUSY_CYCLES"))
            valu = avg(main, lambda i: cval(sq, i, "SQ_INSTS_VALU"))
            mfma = avg(main, lambda i: cval(sq, i, "SQ_INSTS_MFMA"))
            lds_c = avg(main, lambda i: cval(sq, i, "SQ_LDS_BANK_CONFLICT"))
            busy_pct = busy / (1024 * t_main * 1e-6 * 2.4e9) * 100 if busy is not None and t_main else None
            tfl = 2 * M * N * K / ((t_main + t_red) * 1e-6) / 1e12
            fmt = lambda v, p: "-" if v is None else f"{v:.{p}f}"  # noqa: E731
            lines.append(f"| {M} | {name.split('_')[0]} | `{short(trace[main[0]]['Kernel_Name'])}` | {wgs(main[0])} | "
                         f"{t_main:.2f} | {t_red:.2f} | {tfl:.0f} | {fmt(traffic, 1)} | "
                         f"{lin_bytes(N, K, M) / 1e6:.1f} | {fmt(busy_pct, 1)} | "
                         f"{fmt(valu / mfma if valu is not None and mfma else None, 2)} | {fmt(lds_c, 0)} |")
            pos += 52 * L
        L = period(pos, 14, 4)  # the fused block: q/k/v grouped, o, gate/up grouped, down
        passes = [pos + p * L for p in range(14)][-10:]
        pat = seq[pos:pos + L]
        # calls of the pattern: a reduce kernel belongs to the call before it
        starts = [i for i in range(L) if "reduce" not in pat[i][0]]
        for ci, (s0, label) in enumerate(zip(starts, ("q + k + v", "o", "gate + up", "down"))):
            s1 = starts[ci + 1] if ci + 1 < len(starts) else L
            main = [p + s0 for p in passes]
            red = [p + s0 + 1 for p in passes] if s1 - s0 == 2 else []
            t_main = avg(main, dur)
            busy = avg(main, lambda i: cval(sq, i, "SQ_VALU_MFMA_BUSY_CYCLES"))
            busy_pct = busy / (1024 * t_main * 1e-6 * 2.4e9) * 100 if busy is not None and t_main else None
            fused.append(f"| {M} | {label} | `{short(pat[s0][0])}` | {wgs(main[0])} | {t_main:.2f} | "
                         f"{avg(red, dur) if red else 0.0:.2f} | {'-' if busy_pct is None else f'{busy_pct:.1f}'} |")
        pos += 14 * L
    head = []
    if calib:
        head.append(f"- calibration (32 MiB device copy): FETCH_SIZE x {calib.get('FETCH_SIZE', 0):.3f}, "
                    f"WRITE_SIZE x {calib.get('WRITE_SIZE', 0):.3f}")
    return "\n".join(head + ["", "Per linear:", ""] + lines + ["", "Fused block (4 calls):", ""] + fused)


def summarize_grid(d: Path, match: str = "") -> str:
    """Markdown table of a rocprofv3 run directory (``trace/``, ``fetch/``,
    ``write/``, optional ``sq/``) per (kernel, workgroup count): average
    duration, FETCH_SIZE / WRITE_SIZE per dispatch scaled by the same counters
    on the run's 32 MiB device copy (``--copy-calib``), and the other
    counters per dispatch.  ``match``: keep kernels whose name contains it."""
    import csv
    import gzip

    def rows(sub, name):
        fs = sorted((d / sub).glob(f"**/run_{name}.csv*"))
        if not fs:
            return []
        f = fs[0]
        with (gzip.open(f, "rt") if f.suffix == ".gz" else open(f)) as fh:
            return list(csv.DictReader(fh))

    def short(n):
        return n.replace("void ", "").split("(")[0]

    dur = {}
    for r in rows("trace", "kernel_trace"):
        if "w4::" in r["Kernel_Name"] and match in r["Kernel_Name"]:
            key = (short(r["Kernel_Name"]), int(r["Grid_Size_X"]) // int(r["Workgroup_Size_X"]))
            dur.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    calib, ctr = {}, {}
    for sub in ("fetch", "write", "sq"):
        per = {}
        for r in rows(sub, "counter_collection"):
            k = (r["Dispatch_Id"], r["Kernel_Name"], int(r["Grid_Size"]) // int(r["Workgroup_Size"]))
            c = per.setdefault(k, {})
            c[r["Counter_Name"]] = c.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        for (_, kn, wg), cs in sorted(per.items(), key=lambda kv: int(kv[0][0])):
            if "copyBuffer" in kn:
                for cname, v in cs.items():
                    calib.setdefault(cname, 32768.0 / v)
            elif "w4::" in kn and match in kn:
                for cname, v in cs.items():
                    ctr.setdefault((short(kn), wg), {}).setdefault(cname, []).append(v)
    fs, ws = calib.get("FETCH_SIZE"), calib.get("WRITE_SIZE")
    out = [f"- calibration (32 MiB device copy): FETCH_SIZE x {fs or 0:.3f}, WRITE_SIZE x {ws or 0:.3f}", "",
           "| kernel | WGs | dispatches | avg us | FETCH MB | WRITE MB | other counters per dispatch |",
           "|---|---|---|---|---|---|---|"]
    for key in sorted(dur):
        c = ctr.get(key, {})

        def mb(name, scale):
            v = c.get(name)
            return "-" if not v or not scale else f"{sum(v) / len(v) * scale * 1024 / 1e6:.2f}"
        other = ", ".join(f"{n} {sum(v) / len(v):.4g}" for n, v in sorted(c.items())
                          if n not in ("FETCH_SIZE", "WRITE_SIZE"))
        t = dur[key]
        out.append(f"| `{key[0]}` | {key[1]} | {len(t)} | {sum(t) / len(t):.2f} | {mb('FETCH_SIZE', fs)} | "
                   f"{mb('WRITE_SIZE', ws)} | {other} |")
    return "\n".join(out)


def profiled_traffic() -> dict | None:
    """HBM bytes per launch of the roofline kernel, from the committed profile."""
    if not PROFILE.exists():
        return None
    for line in PROFILE.read_text().splitlines():
        if line.startswith("- traffic_bytes_per_launch:"):
            return {"bytes": int(float(line.split(":")[1])), "source": str(PROFILE.relative_to(ROOT))}
    return None


PREFILL_PROFILE = ROOT / "profiles" / "prefill_per_linear_m128_m512_m2048.md"
MFMA_ROOFLINE_LINEAR = "gate"  # M = 2048: gate/up (one kernel, two launches) take the largest share


def profiled_prefill(M: int, linear: str) -> dict | None:
    """Main kernel and HBM bytes per call of one linear of the prefill
    section, from the committed per-linear profile table."""
    if not PREFILL_PROFILE.exists():
        return None
    for line in PREFILL_PROFILE.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 9 and cells[0] == str(M) and cells[1] == linear:
            try:
                traffic = int(float(cells[7]) * 1e6)
            except ValueError:
                traffic = None
            return {"kernel": cells[2].strip("`"), "bytes": traffic, "source": str(PREFILL_PROFILE.relative_to(ROOT))}
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=160)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--sets", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-reps", type=int, default=7, help="timed passes of each CPU baseline (median)")
    ap.add_argument("--cpu-numpy", action="store_true", help="also time the single-core numpy oracle")
    ap.add_argument("--only", default="all",
                    help="comma list of sections to run: decode, perlinear, splitk, prefill, quantize, llama "
                         "(profiling runs use one section; the JSON line needs 'decode')")
    ap.add_argument("--small-m", default="2,4,8,16,32,64",
                    help="comma list of M for the small-M section (profiling runs may pick one)")
    ap.add_argument("--small-g", default="128,64,32", help="comma list of group sizes for the small-M section")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run one 32 MiB device copy (for scaling FETCH_SIZE/WRITE_SIZE counters)")
    ap.add_argument("--summarize-prof", default=None, metavar="DIR",
                    help="print the profile summary of a rocprofv3 run directory and exit (no GPU use)")
    ap.add_argument("--summarize-prefill-prof", default=None, metavar="DIR",
                    help="print the per-linear tables of a rocprofv3 run of --only prefill and exit (no GPU use)")
    ap.add_argument("--summarize-grid", metavar="DIR",
                    help="print per (kernel, workgroup count) times and counters of a rocprofv3 run directory "
                         "and exit (no GPU use)")
    ap.add_argument("--match", default="", help="with --summarize-grid: kernels whose name contains this")
    args = ap.parse_args()
    if args.summarize_prof:
        print(summarize_prof(Path(args.summarize_prof)))
        return 0
    if args.summarize_grid:
        print(summarize_grid(Path(args.summarize_grid), args.match))
        return 0
    if args.summarize_prefill_prof:
        print(summarize_prefill_prof(Path(args.summarize_prefill_prof)))
        return 0
    only = set(args.only.split(",")) if args.only != "all" else {"decode", "perlinear", "splitk", "prefill", "quantize",
                                                                  "llama"}
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the W4A16 path has no collective); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import int4_hip

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(dev)
    nsets = args.sets
    gen = torch.Generator(device=dev).manual_seed(1234)

    # ---------------------------------------------------------------- inputs
    log(f"generating {nsets} weight sets ...")
    w16 = [[(torch.randn((N, K), generator=gen, device=dev) * 0.02).to(torch.bfloat16) for _, N, K in LINEARS]
           for _ in range(nsets)]
    packed = [[int4_hip.quantize_int4(w, G) for w in ws] for ws in w16]
    xs1 = [[torch.randn((1, K), generator=gen, device=dev).to(torch.bfloat16) for _, N, K in LINEARS]
           for _ in range(nsets)]
    ys1 = [[torch.empty((1, N), device=dev, dtype=torch.bfloat16) for _, N, K in LINEARS] for _ in range(nsets)]
    torch.cuda.synchronize()

    if args.copy_calib:
        src = torch.empty(32 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # ------------------------------------------------- quantize kernel (load time)
    q_ms = q7_ms = None
    q_bytes = sum(2 * N * K + N * K // 2 + 4 * N * K // G for _, N, K in LINEARS)
    if "quantize" in only:
        # the block's 7 weights as one grouped launch (w4_quantize_grouped),
        # and as 7 launches (one quantize_int4 per linear, the reference's
        # per-module conversion)
        def quant_set(i):
            return lambda: int4_hip.quantize_int4_grouped(w16[i], G)

        def quant_set7(i):
            return lambda: [int4_hip.quantize_int4(w, G) for w in w16[i]]

        gq = graph_of(lambda: [quant_set(i)() for i in range(nsets)], stream)
        q_ms = time_graph(gq, 3, stream) / nsets
        del gq
        gq7 = graph_of(lambda: [quant_set7(i)() for i in range(nsets)], stream)
        q7_ms = time_graph(gq7, 3, stream) / nsets
        del gq7
    # the first set's bf16 weights, kept on the host for the CPU quantize baseline
    w16_host = [w.cpu() for w in w16[0]] if ("quantize" in only and not args.no_cpu) else None
    del w16
    torch.cuda.empty_cache()

    # ------------------------------------------------- M=1 decode block: grouped launch
    def grouped(i):
        return lambda: int4_hip.w4a16_matmul_grouped(xs1[i], packed[i], out=ys1[i])

    steps, warm = args.steps, args.warmup
    bytes1 = block_bytes(1)
    ms_per_step = kern_ms = value = achieved = steady_ms = None
    kern_ms_src = None
    if "decode" in only:
        # Exactly `warm` untimed steps, then exactly `steps` timed ones, each
        # step one call of the library's grouped entry point (the one
        # w4a16_matmul_grouped makes) on weight set i % nsets, issued back to
        # back from a C loop (csrc/bench/launch_loop.cpp) so that the GPU, not
        # the interpreter, sets the pace; HIP events on the launch stream
        # bracket the timed calls, host synchronisation on both sides.
        import ctypes

        lib = int4_hip._lib.load()
        blib_path = ROOT / "itmo-final-project_amd" / "int4_hip" / "libw4_bench.so"
        nprob = len(LINEARS)
        probs = (int4_hip._lib.Problem * (nprob * nsets))()
        for i in range(nsets):
            for j, (x, (qw, sc, ze), y) in enumerate(zip(xs1[i], packed[i], ys1[i])):
                K = x.shape[1]
                probs[i * nprob + j] = int4_hip._lib.Problem(x.data_ptr(), qw.data_ptr(), sc.data_ptr(), ze.data_ptr(),
                                                             y.data_ptr(), qw.shape[1], K, K // sc.shape[0], 0)
        ws_need = lib.w4a16_grouped_workspace_bytes(probs, nprob, 1)
        ws = int4_hip.gemm._stream_workspace(dev, stream.cuda_stream, ws_need) if ws_need else None
        ws_ptr, ws_len = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
        fn_ptr = ctypes.cast(lib.w4a16_gemm_grouped, ctypes.c_void_p).value
        blib = ctypes.CDLL(str(blib_path)) if blib_path.exists() else None
        if blib is not None:
            loop = blib.w4bench_grouped_steps
            loop.restype = ctypes.c_int
            loop.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                             ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p,
                             ctypes.c_size_t, ctypes.c_void_p]

            def c_steps(first, n):
                # steps first .. first + n - 1 of the rotation over the weight sets
                rc = loop(fn_ptr, ctypes.cast(probs, ctypes.c_void_p), ctypes.sizeof(int4_hip._lib.Problem) * nprob,
                          nprob, nsets, first, n, int4_hip._lib.DTYPE_BF16, 1, ws_ptr, ws_len, stream.cuda_stream)
                if rc != 0:
                    raise RuntimeError(f"w4a16_gemm_grouped failed in the step loop ({rc})")

            blib.w4bench_gate_new.restype = ctypes.c_void_p
            blib.w4bench_gate_close.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_double]
            blib.w4bench_gate_open.argtypes = [ctypes.c_void_p]
            blib.w4bench_gate_state.argtypes = [ctypes.c_void_p]
            blib.w4bench_gate_free.argtypes = [ctypes.c_void_p]
            blib.w4bench_event_new.restype = ctypes.c_void_p
            blib.w4bench_event_record.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            blib.w4bench_event_ms.restype = ctypes.c_double
            blib.w4bench_event_ms.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            blib.w4bench_event_free.argtypes = [ctypes.c_void_p]
            gate = blib.w4bench_gate_new()
            ev0, ev1 = blib.w4bench_event_new(), blib.w4bench_event_new()
            if not (gate and ev0 and ev1):
                raise RuntimeError("bench: could not create the step gate or the timing events")
            c_steps(0, warm)
            torch.cuda.synchronize()
            # the gate holds the stream until every timed call is queued, so
            # the events bracket the GPU's back-to-back execution of the steps
            # and not the host's latency to issue the first of them; the
            # events are timing-only (no system-scope fence when recorded)
            if blib.w4bench_gate_close(gate, stream.cuda_stream, 500.0) != 0:
                raise RuntimeError("bench: step gate launch failed")
            blib.w4bench_event_record(ev0, stream.cuda_stream)
            c_steps(warm, steps)  # the rotation continues: no set is read twice within 16 steps
            blib.w4bench_event_record(ev1, stream.cuda_stream)
            blib.w4bench_gate_open(gate)
            torch.cuda.synchronize()
            gate_state = blib.w4bench_gate_state(gate)
            ms_run = blib.w4bench_event_ms(ev0, ev1)
            for h in (ev0, ev1):
                blib.w4bench_event_free(h)
            blib.w4bench_gate_free(gate)
            if ms_run <= 0:
                raise RuntimeError("bench: reading the timing events failed")
            kern_ms_src = ("hip-events-on-launch-stream-over-the-timed-steps (C loop of C-ABI calls, queued "
                           "behind a host-opened gate" + ("" if gate_state == 2 else ", gate timed out") +
                           "; events without the system-scope fence)")
        else:  # no bench helper: the timed steps as one graph replay
            with torch.cuda.stream(stream):
                for i in range(warm):
                    grouped(i % nsets)()
            torch.cuda.synchronize()
            g_steps = graph_of(lambda: [grouped((warm + i) % nsets)() for i in range(steps)], stream,
                               eager_warmup=False)
            ms_run = time_graph_once(g_steps, stream)
            del g_steps
            kern_ms_src = "hip-events-on-launch-stream-over-the-timed-steps (one graph replay)"
        ms_per_step = ms_run / steps
        value = bytes1 / (ms_per_step * 1e-3) / 1e9
        # one kernel per step: the roofline kernel's average duration is the
        # timed region over its launches
        kern_ms = ms_per_step
        achieved = bytes1 / (kern_ms * 1e-3) / 1e9
        # steady state beside it: a graph of the 16 sets replayed back to back
        # (median of five runs of 10 replays, so one disturbed run does not set it)
        g_main = graph_of(lambda: [grouped(i)() for i in range(nsets)], stream)
        time_graph(g_main, 2, stream)
        steady_ms = sorted(time_graph(g_main, 10, stream) for _ in range(5))[2] / nsets
        del g_main

    # ------------------------------------------------- M=1 per-linear launches (reference-comparable)
    def single(i, j):
        return lambda: int4_hip.w4a16_matmul(xs1[i][j], *packed[i][j])

    per_lin, ms7, ms4, resident = {}, None, None, None
    if "perlinear" in only:
        for j, (name, N, K) in enumerate(LINEARS):
            gj = graph_of(lambda j=j: [single(i, j)() for i in range(nsets)], stream)
            time_graph(gj, 2, stream)
            per_lin[name] = time_graph(gj, 10, stream) / nsets * 1e3
            del gj
        g7 = graph_of(lambda: [single(i, j)() for i in range(nsets) for j in range(len(LINEARS))], stream)
        time_graph(g7, 2, stream)
        ms7 = time_graph(g7, 10, stream) / nsets
        del g7
        # the block as a decoder issues it (4 calls: q/k/v and gate/up share an input)
        g4 = graph_of(lambda: [f for i in range(nsets) for f in (
            int4_hip.w4a16_matmul_grouped([xs1[i][0]] * 3, packed[i][0:3]),
            int4_hip.w4a16_matmul(xs1[i][3], *packed[i][3]),
            int4_hip.w4a16_matmul_grouped([xs1[i][4]] * 2, packed[i][4:6]),
            int4_hip.w4a16_matmul(xs1[i][6], *packed[i][6]))], stream)
        time_graph(g4, 2, stream)
        ms4 = time_graph(g4, 10, stream) / nsets
        del g4
        # cache-resident figures (one weight set, 32 MB, replayed: it stays in
        # the 256 MB Infinity Cache), comparable to L2-resident numbers
        gr = graph_of(lambda: [grouped(0)() for _ in range(nsets)], stream)
        time_graph(gr, 2, stream)
        resident = {"grouped_us_per_block": time_graph(gr, 10, stream) / nsets * 1e3}
        del gr
        g7r = graph_of(lambda: [single(0, j)() for _ in range(nsets) for j in range(len(LINEARS))], stream)
        time_graph(g7r, 2, stream)
        resident["seven_launches_us_per_block"] = time_graph(g7r, 10, stream) / nsets * 1e3
        del g7r

    # ------------------------------------------------- small-M regime
    # M in {2..64} x G in {128, 64, 32}, per-linear launches over the rotated
    # weight sets (G=128 reuses the decode sets; G=64/32 are quantized here)
    ms16, small = None, {}
    if "splitk" in only:
        for g in [int(v) for v in args.small_g.split(",")]:
            if g == G:
                packs = packed
            else:
                packs = []
                for _ in range(nsets):
                    one = []
                    for _, N, K in LINEARS:
                        w = (torch.randn((N, K), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
                        one.append(int4_hip.quantize_int4(w, g))
                        del w
                    packs.append(one)
            small[g] = {}
            for M in [int(v) for v in args.small_m.split(",")]:
                xsm = [torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16) for _, N, K in LINEARS]
                gm = graph_of(lambda: [int4_hip.w4a16_matmul(xsm[j], *packs[i][j]) for i in range(nsets)
                                       for j in range(len(LINEARS))], stream)
                time_graph(gm, 2, stream)
                msm = time_graph(gm, 5, stream) / nsets
                small[g][M] = {"us_per_block": round(msm * 1e3, 2),
                               "gbps": round(block_bytes(M, g) / (msm * 1e-3) / 1e9, 1)}
                if g == G and M == 16:
                    ms16 = msm
                del gm
                if M <= 64:
                    # all seven products in one launch (as the M=1 headline figure)
                    gg = graph_of(lambda: [int4_hip.w4a16_matmul_grouped(xsm, packs[i]) for i in range(nsets)],
                                  stream)
                    time_graph(gg, 2, stream)
                    msg = time_graph(gg, 5, stream) / nsets
                    small[g][M]["grouped_us_per_block"] = round(msg * 1e3, 2)
                    small[g][M]["grouped_gbps"] = round(block_bytes(M, g) / (msg * 1e-3) / 1e9, 1)
                    del gg
                if g == G:
                    # the block as a model issues it: q/k/v and gate/up share an input
                    gf = graph_of(lambda: [f for i in range(nsets) for f in (
                        int4_hip.w4a16_matmul_grouped([xsm[0]] * 3, packs[i][0:3]),
                        int4_hip.w4a16_matmul(xsm[3], *packs[i][3]),
                        int4_hip.w4a16_matmul_grouped([xsm[4]] * 2, packs[i][4:6]),
                        int4_hip.w4a16_matmul(xsm[6], *packs[i][6]))], stream)
                    time_graph(gf, 2, stream)
                    msf = time_graph(gf, 5, stream) / nsets
                    small[g][M]["fused_qkv_gateup_us_per_block"] = round(msf * 1e3, 2)
                    small[g][M]["fused_qkv_gateup_gbps"] = round(block_bytes(M, g) / (msf * 1e-3) / 1e9, 1)
                    del gf
                del xsm
            if g != G:
                del packs
            torch.cuda.empty_cache()

    # ------------------------------------------------- prefill M=128/512/2048
    pre = {}
    if "prefill" in only:
        for M in (128, 512, 2048):
            xsM = [torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16) for _, N, K in LINEARS]
            gp = graph_of(lambda: [int4_hip.w4a16_matmul(xsM[j], *packed[0][j]) for j in range(len(LINEARS))],
                          stream)
            time_graph(gp, 3, stream)
            msM = time_graph(gp, 10, stream)
            pre[M] = {"us_per_block": round(msM * 1e3, 2), "tflops": round(block_flops(M) / (msM * 1e-3) / 1e12, 2)}
            del gp
            per = {}
            for j, (name, N, K) in enumerate(LINEARS):
                gj = graph_of(lambda j=j: [int4_hip.w4a16_matmul(xsM[j], *packed[0][j]) for _ in range(4)], stream)
                time_graph(gj, 2, stream)
                per[name] = round(time_graph(gj, 10, stream) / 4 * 1e3, 2)
                del gj
            pre[M]["per_linear_us"] = per
            # the same block with the projections that share an input fused
            # (q/k/v and gate/up as grouped calls): 4 W4A16 calls instead of 7
            gf = graph_of(lambda: [int4_hip.w4a16_matmul_grouped([xsM[0]] * 3, packed[0][0:3]),
                                   int4_hip.w4a16_matmul(xsM[3], *packed[0][3]),
                                   int4_hip.w4a16_matmul_grouped([xsM[4]] * 2, packed[0][4:6]),
                                   int4_hip.w4a16_matmul(xsM[6], *packed[0][6])], stream)
            time_graph(gf, 3, stream)
            msf = time_graph(gf, 10, stream)
            pre[M]["fused_qkv_gateup_us_per_block"] = round(msf * 1e3, 2)
            pre[M]["fused_qkv_gateup_tflops"] = round(block_flops(M) / (msf * 1e-3) / 1e12, 2)
            del gf
            w_deq = [int4_hip.dequantize_int4(*packed[0][j], torch.bfloat16) for j in range(len(LINEARS))]
            gb = graph_of(lambda: [torch.nn.functional.linear(xsM[j], w_deq[j]) for j in range(len(LINEARS))],
                          stream)
            time_graph(gb, 3, stream)
            msb = time_graph(gb, 10, stream)
            pre[M]["hipblaslt_bf16_dequantized_us"] = round(msb * 1e3, 2)
            pre[M]["hipblaslt_bf16_tflops"] = round(block_flops(M) / (msb * 1e-3) / 1e12, 2)
            del gb, w_deq
            del xsM
    torch.cuda.synchronize()

    # ---------------------------- end to end: random-init Llama-3.2-1B with Int4Linear
    llama = None
    if "llama" in only:
        from int4_hip.llama import run_eval
        log("llama: 512-token prefill + 128 graph decode steps, bf16 then W4 ...")
        try:
            llama = run_eval(prompt_len=512, new_tokens=128, group_size=G)
            llama.pop("config", None)
            # the reference's --quantize-lm-head variant (untied, 128256 x 2048 lm_head in int4)
            lm = run_eval(prompt_len=512, new_tokens=128, group_size=G, quantize_lm_head=True, reps=2)
            llama["quantize_lm_head"] = {k: lm[k] for k in (
                "linear_weight_bytes", "model_bytes", "w4_prefill_tokens_per_s", "w4_decode_tokens_per_s",
                "w4_decode_ms_per_token", "vs_fake_prefill_top1_agreement", "vs_fake_prefill_kl_mean")}
        except Exception as e:  # reported in the line; the kernel figures above stand
            llama = {"error": repr(e)[:400]}
        torch.cuda.synchronize()

    # ------------------------------------------------- CPU baseline (rank 0, N=1)
    cpu = cpu_q = cpu_np = None
    if not args.no_cpu:
        def bits(t):
            return t.contiguous().view(torch.int16).numpy().view(np.uint16)
        packed0 = [tuple(t.cpu() for t in p) for p in packed[0]]
        xs0 = [x.cpu() for x in xs1[0]]
        cpu = cpu_baseline(packed0, xs0, args.cpu_reps)
        if args.cpu_numpy:
            cpu_np = cpu_numpy_port([(qw.numpy(), bits(sc), bits(ze)) for qw, sc, ze in packed0],
                                    [bits(x) for x in xs0], 3)
        if "quantize" in only:
            cpu_q = cpu_quantize_baseline(w16_host, q_bytes, args.cpu_reps)
    copy_gbps = device_copy_gbps(dev, stream) if "decode" in only else None
    read_ceiling = hbm_read_ceiling(dev, stream, bytes1, nsets) if "decode" in only else None

    traffic = profiled_traffic()
    # the M = 2048 half of the metric: the dominant prefill kernel against the
    # bf16 MFMA peak (its per-call time from the section's graph of 4 lone
    # calls, timed with events on the launch stream; its traffic from the
    # committed per-linear profile)
    pre_roof = None
    if pre:
        name = MFMA_ROOFLINE_LINEAR + "_proj"
        _, N, K = next(lin for lin in LINEARS if lin[0] == name)
        t_us = pre[2048]["per_linear_us"][name]
        ach = 2 * 2048 * N * K / (t_us * 1e-6) / 1e12
        prof = profiled_prefill(2048, MFMA_ROOFLINE_LINEAR)
        pre_roof = {"bound": "mfma", "linear": name, "M": 2048,
                    "kernel": ("w4::" + prof["kernel"].replace("w4::", "")) if prof else None,
                    "kernel_us": t_us, "achieved": round(ach, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(ach / MFMA_BF16_PEAK_TFLOPS, 4),
                    "traffic": prof["bytes"] if prof else None, "traffic_source": prof["source"] if prof else None,
                    "algorithmic_bytes": lin_bytes(N, K, 2048),
                    "kernel_time_source": "hip-events-on-launch-stream over 10 graph replays of 4 lone calls"}
    out = {
        "metric": METRIC,
        "value": round(value, 2) if value is not None else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": round(ms_per_step, 6) if ms_per_step is not None else None,
        "us_per_block": round(ms_per_step * 1e3, 3) if ms_per_step is not None else None,
        "us_per_block_steady_replays": round(steady_ms * 1e3, 3) if steady_ms is not None else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "Llama-3.2-1B decoder block: 7 W4A16 linears (q/k/v/o/gate/up/down), M=1 "
                               "decode GEMV as one grouped launch, G=128, bf16 activations, "
                               f"{nsets} rotated weight sets ({nsets * bytes1 / 1e6:.0f} MB)",
                   "M": 1, "group_size": G, "weight_sets": nsets, "bytes_per_step": bytes1},
        "roofline": None if achieved is None else {
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic["bytes"] if traffic else None,
            "traffic_source": traffic["source"] if traffic else None,
            "kernel": "w4::" + ROOFLINE_KERNEL, "kernel_us": round(kern_ms * 1e3, 3),
            "kernel_time_source": kern_ms_src},
        "cpu_baseline": cpu,
        "cpu_baseline_numpy_port": cpu_np,
        "decode_m1_per_linear_us": {k: round(v, 3) for k, v in per_lin.items()},
        "decode_m1_per_linear_gbps": {name: round(lin_bytes(N, K) / (per_lin[name] * 1e-6) / 1e9, 1)
                                      for name, N, K in LINEARS if name in per_lin},
        "decode_m1_cache_resident": None if resident is None else {
            k: round(v, 3) for k, v in resident.items()},
        "decode_m1_7_launches_us_per_block": round(ms7 * 1e3, 3) if ms7 else None,
        "decode_m1_7_launches_gbps": round(bytes1 / (ms7 * 1e-3) / 1e9, 1) if ms7 else None,
        "decode_m1_4_calls_us_per_block": round(ms4 * 1e3, 3) if ms4 else None,
        "decode_m1_4_calls_gbps": round(bytes1 / (ms4 * 1e-3) / 1e9, 1) if ms4 else None,
        "small_m_7_launches": {f"G{g}": {f"M{m}": v for m, v in d.items()} for g, d in small.items()},
        "splitk_m16_us_per_block": round(ms16 * 1e3, 3) if ms16 else None,
        "splitk_m16_gbps": round(block_bytes(16) / (ms16 * 1e-3) / 1e9, 1) if ms16 else None,
        "prefill": {str(k): v for k, v in pre.items()},
        "prefill_m2048_tflops": pre[2048]["tflops"] if pre else None,
        "prefill_m2048_mfma_frac": round(pre[2048]["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4) if pre else None,
        "prefill_m2048_roofline": pre_roof,
        "quantize_us_per_block": round(q_ms * 1e3, 2) if q_ms else None,
        "quantize_gbps": round(q_bytes / (q_ms * 1e-3) / 1e9, 1) if q_ms else None,
        "quantize_7_launches_us_per_block": round(q7_ms * 1e3, 2) if q7_ms else None,
        "cpu_baseline_quantize": cpu_q,
        "hbm_device_copy_gbps": round(copy_gbps, 1) if copy_gbps else None,
        "hbm_read_ceiling": read_ceiling,
        "llama_1b_w4": llama,
        "device": torch.cuda.get_device_name(dev),
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
