#!/usr/bin/env python3
"""Benchmark of the fused GGUF SoA dequantize + GEMV on one MI355X.

Headline (the JSON line's `value`): HBM GB/s of the Q5_0 GEMV sweep over the
StarCoder2-8B decoder linears at batch (beam) 2: fused qkv 5632x4608, o_proj
4608x4608, c_fc 18432x4608, c_proj 4608x18432 and lm_head 49152x4608. One step
is one pass over the five matrices (one GEMV each); `value` = algorithmic
bytes per step / time per step, where algorithmic bytes = packed weights +
scales + fp16 x + fp16 y + fp16 bias.

Measurement: seeded synthetic weights resident in HBM. Every matrix exists in
8 distinct copies (>= 2.4 GB per pass rotation), so each launch reads weights
that the 256 MB Infinity Cache no longer holds; step i uses copy i % 8. After
exactly W untimed steps, a HIP graph of exactly K steps is replayed in 5
trials, each bracketed by HIP events on the launch stream and device
synchronization; `value` is from the median trial. The `roofline` object is
for the dominant launch (lm_head), timed the same way in its own graph.
`sweep` holds every GEMV configuration (1B Q4_0 shapes, 8B Q5_0 shapes,
8192x2048 Q8_0, the beam-width sweep), each as the median of 5 trials over
>= 1 GiB of rotating copies. `cpu_baseline` times the reference's CPU path
(tiled fp32 dequantize + F.linear, restated in oracle/) on the host cores for
one pass of the same step, and `cpu_sweep` every sweep configuration.
`decode` holds the decode loops: the StarCoder2-8B-style loop (32 layers,
Q4_0, beam 2) and the GPTBigCode-1B loop (24 layers, Q4_0 linears, Q8_0
tables, beam 2), each run as the reference specifies it (torch attention,
LayerNorm and sampling around the HIP GEMVs) and fused.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--quick]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402
import torch  # noqa: E402

import __graft_entry__  # noqa: E402

__graft_entry__.register_package()
import starvector_amd._native as native  # noqa: E402
from starvector_amd.quantization import BLOCK_BYTES  # noqa: E402

PEAK_HBM_GBS = 8000.0
METRIC = "quant GEMV HBM GB/s (% of peak) at 8B shapes; 8B beam-2 decode tokens/s"
STEP_SHAPES = [  # (name, n, k, has_bias) of the 8B decoder step, Q5_0, batch 2
    ("qkv", 5632, 4608, True), ("o_proj", 4608, 4608, True), ("c_fc", 18432, 4608, True),
    ("c_proj", 4608, 18432, True), ("lm_head", 49152, 4608, False)]
STEP_QTYPE, STEP_M, COPIES = "Q5_0", 2, 8


KERNEL_NAMES = {"stream": "svq::gemv_stream_kernel", "chunked": "svq::gemv_kernel",
                "mfma": "svq::gemv_mfma_kernel", "mfma4": "svq::gemv_mfma4_kernel"}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def algorithmic_bytes(qtype, n, k, m, bias):
    return n * k // 32 * BLOCK_BYTES[qtype] + 2 * m * k + 2 * m * n + (2 * n if bias else 0)


class Pool:
    """Distinct weight copies carved from two large seeded device buffers."""

    def __init__(self, dev, q_bytes, s_bytes, seed=1234):
        g = torch.Generator(device=dev).manual_seed(seed)
        self.q = torch.randint(0, 256, (q_bytes,), dtype=torch.uint8, device=dev, generator=g)
        d = torch.rand(s_bytes // 2, device=dev, generator=g) * (2e-2 - 1e-3) + 1e-3
        self.s = d.half().view(torch.uint8)
        self.dev = dev
        self.reset()

    def reset(self):
        """Start carving from the beginning of the pool again."""
        self.q_cursor = self.s_cursor = 0

    def copies(self, qtype, n, k, count):
        """`count` copies at pool regions disjoint from every copy taken since
        the last reset()."""
        blocks = n * k // 32
        qb = blocks * (BLOCK_BYTES[qtype] - 2)
        sb = blocks * 2
        align = lambda v: (v + 255) // 256 * 256
        out = []
        for i in range(count):
            qo, so = self.q_cursor, self.s_cursor
            self.q_cursor += align(qb)
            self.s_cursor += align(sb)
            if qo + qb > self.q.numel() or so + sb > self.s.numel():
                raise ValueError("pool too small")
            q = self.q[qo:qo + qb]
            if qtype == "Q8_0":  # keep codes in [-127, 127] as the benchmark specifies
                q = q.clone()
                q[q == 0x80] = 0x81
            out.append((q, self.s[so:so + sb].view(torch.float16)))
        return out


def copies_for(nbytes, cap_bytes):
    return max(2, min(int(math.ceil(2**30 / nbytes)), cap_bytes // nbytes))


def make_call(x, q, s, y, qtype, bias):
    """One GEMV launch as quantization.soa_gemv makes it: with the per-stream
    workspace that lets long rows split K (allocated at the warm-up call,
    before any capture)."""
    m, k = x.shape
    n = y.shape[1]
    return lambda: native.gemv(x, q, s.view(torch.uint8), y, qtype, bias,
                               native.split_workspace(x.device, m, n, k, qtype))


def capture(fns, stream):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        for f in fns:  # warm-up outside capture
            f()
        stream.synchronize()
        with torch.cuda.graph(g, stream=stream):
            for f in fns:
                f()
    return g


def time_graph(graph, stream, replays):
    """Milliseconds per replay, HIP events on the launch stream."""
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):  # replay() launches on the current stream
        start.record(stream)
        for _ in range(replays):
            graph.replay()
        stop.record(stream)
    stop.synchronize()
    return start.elapsed_time(stop) / replays


def gemv_case(pool, dev, stream, qtype, n, k, m, bias, trials=5, replays=3):
    """Median µs per launch over >= 1 GiB of rotating copies."""
    nbytes = algorithmic_bytes(qtype, n, k, m, bias)
    count = copies_for(n * k // 32 * BLOCK_BYTES[qtype], pool.q.numel() // 2)
    pool.reset()
    cps = pool.copies(qtype, n, k, count)
    gen = torch.Generator(device=dev).manual_seed(n + k + m)
    x = torch.randn((m, k), device=dev, generator=gen).half()
    b = torch.randn(n, device=dev, generator=gen).half() if bias else None
    y = torch.empty((m, n), dtype=torch.float16, device=dev)
    graph = capture([make_call(x, q, s, y, qtype, b) for q, s in cps], stream)
    time_graph(graph, stream, 1)
    ms = [time_graph(graph, stream, replays) / count for _ in range(trials)]
    us = statistics.median(ms) * 1e3
    del graph
    return {"qtype": qtype, "n": n, "k": k, "m": m, "bias": bias, "copies": count,
            "us": round(us, 3), "gbs": round(nbytes / us / 1e3, 1),
            "frac": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4), "bytes": nbytes}


def dequant_case(pool, dev, stream, qtype, out_dtype, n=18432, k=4608, trials=5, replays=3):
    """`svq_dequant` of an n x k matrix (quantization.py:93-105 on the GPU):
    median µs per launch over rotating weight copies, algorithmic bytes
    (payload + scales read, output written)."""
    blocks = n * k // 32
    out_bytes = torch.tensor([], dtype=out_dtype).element_size() * n * k
    nbytes = blocks * BLOCK_BYTES[qtype] + out_bytes
    count = copies_for(blocks * BLOCK_BYTES[qtype], pool.q.numel() // 2)
    pool.reset()
    cps = pool.copies(qtype, n, k, count)
    out = torch.empty((n, k), dtype=out_dtype, device=dev)
    calls = [(lambda q=q, s=s: native.dequant(q, s.view(torch.uint8), out, qtype)) for q, s in cps]
    graph = capture(calls, stream)
    time_graph(graph, stream, 1)
    ms = [time_graph(graph, stream, replays) / count for _ in range(trials)]
    us = statistics.median(ms) * 1e3
    del graph
    return {"qtype": qtype, "n": n, "k": k, "out": str(out_dtype).replace("torch.", ""),
            "us": round(us, 3), "gbs": round(nbytes / us / 1e3, 1),
            "frac": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4), "bytes": nbytes}


def sweep_cases():
    cases = [("cfg1", "Q8_0", 8192, 2048, 1, True)]
    for n, k in ((2304, 2048), (2048, 2048), (8192, 2048), (2048, 8192), (49152, 2048)):
        for m in (1, 2):
            cases.append(("cfg2", "Q4_0", n, k, m, n != 49152))
    for name, n, k, bias in STEP_SHAPES:
        cases.append(("cfg3", "Q5_0", n, k, 2, bias))
    for qtype in ("Q4_0", "Q5_0", "Q8_0"):
        for n, k, bias in ((18432, 4608, True), (49152, 4608, False)):
            for m in (1, 2, 4, 8):
                cases.append(("cfg4", qtype, n, k, m, bias))
    return cases


def profile_pass(dev, stream):
    """Eager launches, one dispatch per GEMV, for kernel traces and counters."""
    pool = Pool(dev, q_bytes=3 * 2**30, s_bytes=2**29)
    gen = torch.Generator(device=dev).manual_seed(0)
    xs = {k: torch.randn((STEP_M, k), device=dev, generator=gen).half() for k in (4608, 18432)}
    calls = {}
    for name, n, k, bias in STEP_SHAPES:
        cps = pool.copies(STEP_QTYPE, n, k, COPIES)
        b = torch.randn(n, device=dev, generator=gen).half() if bias else None
        y = torch.empty((STEP_M, n), dtype=torch.float16, device=dev)
        calls[name] = [make_call(xs[k], q, s, y, STEP_QTYPE, b) for q, s in cps]
    with torch.cuda.stream(stream):
        for _ in range(2):
            for i in range(COPIES):
                for name, *_ in STEP_SHAPES:
                    calls[name][i]()
        stream.synchronize()
        src = torch.empty(2**28, dtype=torch.uint8, device=dev)
        dst = [torch.empty_like(src) for _ in range(4)]
        for i in range(16):
            dst[i % 4].copy_(src)
        stream.synchronize()
    log(f"profile pass done: {2 * COPIES * len(STEP_SHAPES)} GEMV dispatches, 16 copies of {2**28} bytes")


def _is_gemv(name):
    return name.startswith("void svq::") and "gemv" in name


def _is_split_finish(name):
    """Second kernel of a K split across workgroups (part of the GEMV before it)."""
    return "split_finish_kernel" in name


def _fold_split_finish(rows, key="Kernel_Name"):
    """GEMV dispatches in launch order, each K-split GEMV with its finish
    kernel attached under "_finish"."""
    out = []
    for r in rows:
        if _is_split_finish(r[key]) and out:
            out[-1] = dict(out[-1], _finish=r)
        elif _is_gemv(r[key]):
            out.append(r)
    return out


def _short_kernel(name):
    for junk in ("void svq::", "(anonymous namespace)::", "(svq::GemvArgs)"):
        name = name.replace(junk, "")
    return name


def _grid(r):
    """Launch shape of a trace row: total threads, and slices x workgroups when 2-D."""
    x, y, z = (int(r[f"Grid_Size_{a}"]) for a in "XYZ")
    if y == 1 and z == 1:
        return str(x)
    return f"{x * y * z} ({x // int(r['Workgroup_Size_X'])}x{y * z} wg)"


def _read_csv(path):
    import csv
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _durations_us(rows):
    """Kernel durations; a K-split GEMV counts both of its kernels."""
    def one(r):
        return (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    return [one(r) + (one(r["_finish"]) if "_finish" in r else 0.0) for r in rows]


def _counter_dispatches(path):
    """{correlation id: (kernel name, {counter: value summed over its instances})}, in order."""
    per = {}
    for r in _read_csv(path):
        name, c = per.setdefault(r["Correlation_Id"], (r["Kernel_Name"], {}))
        c[r["Counter_Name"]] = c.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return [per[key] for key in sorted(per, key=int)]


def summarize(root: Path):
    """Tables from rocprofv3 CSV output found under `root`.

    * A kernel trace of `bench.py --profile` (two eager passes of the step on
      8 weight copies) is tabulated per step shape: GEMV dispatches are mapped
      to shapes by their launch order. Any other kernel trace (for instance
      of the plain bench command) is grouped by kernel, grid and LDS size.
    * Counter collections of `bench.py --profile` are averaged per shape. The
      torch copy of 256 MiB is the plain copy kernel of known size: FETCH_SIZE
      and WRITE_SIZE (KiB per dispatch) are scaled by 256 MiB / what the copy
      reads for them, and a "traffic" line per shape gives the HBM bytes per
      launch that result, next to the algorithmic bytes.
    """
    shapes = list(STEP_SHAPES)
    profile_dispatches = 2 * COPIES * len(shapes)
    copy_kib = 2**28 / 1024
    out = []
    for trace in sorted(root.rglob("*kernel_trace.csv")):
        # Rows are written as dispatches complete; launch order is Dispatch_Id.
        rows = sorted(_read_csv(trace), key=lambda r: int(r["Dispatch_Id"]))
        gemv = _fold_split_finish(rows)
        copies = [r for r in rows if "copyBuffer" in r["Kernel_Name"]]
        out.append(f"kernel trace: {trace.relative_to(root)} ({len(gemv)} GEMV dispatches)")
        if len(gemv) == profile_dispatches:
            out.append("| shape | kernel | grid | VGPR | LDS B | dispatches | avg us | min us "
                       "| GB/s (algorithmic) | % of 8 TB/s |")
            out.append("|---|---|---|---|---|---|---|---|---|---|")
            for i, (name, n, k, bias) in enumerate(shapes):
                mine = gemv[i::len(shapes)]
                durs = _durations_us(mine)
                avg = sum(durs) / len(durs)
                nbytes = algorithmic_bytes(STEP_QTYPE, n, k, STEP_M, bias)
                kname = _short_kernel(mine[0]["Kernel_Name"])
                if "_finish" in mine[0]:
                    kname += " + split_finish_kernel"
                out.append(f"| {name} {n}x{k} | {kname} | "
                           f"{_grid(mine[0])} | {mine[0]['VGPR_Count']} | "
                           f"{mine[0]['LDS_Block_Size']} | {len(mine)} | {avg:.2f} | {min(durs):.2f} | "
                           f"{nbytes / avg / 1e3:.0f} | {nbytes / avg / 1e3 / PEAK_HBM_GBS:.1%} |")
        else:
            groups = {}
            for r in gemv:
                key = (_short_kernel(r["Kernel_Name"]), _grid(r), r["LDS_Block_Size"])
                groups.setdefault(key, []).append(r)
            out.append("| kernel | grid | LDS B | dispatches | avg us | min us | max us |")
            out.append("|---|---|---|---|---|---|---|")
            for (kname, grid, lds), mine in groups.items():
                durs = _durations_us(mine)
                out.append(f"| {kname} | {grid} | {lds} | {len(mine)} | {sum(durs) / len(durs):.2f} | "
                           f"{min(durs):.2f} | {max(durs):.2f} |")
        if copies and len(gemv) == profile_dispatches:
            durs = _durations_us(copies)
            out.append(f"| torch copy 256 MiB | {_grid(copies[0])} | | {len(copies)} | "
                       f"{sum(durs) / len(durs):.2f} | {min(durs):.2f} | "
                       f"{2 * 2**28 / (sum(durs) / len(durs)) / 1e3:.0f} GB/s read+write |")
        out.append("")
    for stats in sorted(root.rglob("*kernel_stats.csv")):
        out.append(f"kernel stats (rocprofv3 --stats): {stats.relative_to(root)}")
        out.append("| kernel | calls | avg us | min us | max us | % of GPU time |")
        out.append("|---|---|---|---|---|---|")
        for r in _read_csv(stats):
            if _is_gemv(r["Name"]) or _is_split_finish(r["Name"]) or "copyBuffer" in r["Name"]:
                out.append(f"| {_short_kernel(r['Name'])} | {r['Calls']} | "
                           f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                           f"{float(r['MaxNs']) / 1e3:.2f} | {r['Percentage']} |")
        out.append("")
    per_shape = {}   # shape name -> {counter: average per dispatch}
    scale = {}       # counter -> bytes per unit the counter reports
    for coll in sorted(root.rglob("*counter_collection.csv")):
        disp = _counter_dispatches(coll)
        gemv = []
        for name, c in disp:  # a K split's finish kernel adds to its GEMV
            if _is_split_finish(name) and gemv:
                gemv[-1] = {key: gemv[-1].get(key, 0.0) + c.get(key, 0.0)
                            for key in set(gemv[-1]) | set(c)}
            elif _is_gemv(name):
                gemv.append(c)
        copies = [c for name, c in disp if "copyBuffer" in name]
        names = sorted({n for c in gemv + copies for n in c})
        out.append(f"counters: {coll.relative_to(root)}")
        out.append("| shape | " + " | ".join(names) + " |")
        out.append("|---|" + "---|" * len(names))
        if len(gemv) == profile_dispatches:
            for i, (name, n, k, bias) in enumerate(shapes):
                mine = gemv[i::len(shapes)]
                vals = {c: sum(d.get(c, 0.0) for d in mine) / len(mine) for c in names}
                per_shape.setdefault(name, {}).update(vals)
                out.append(f"| {name} {n}x{k} | " + " | ".join(f"{vals[c]:.6g}" for c in names) + " |")
        if copies:
            vals = {c: sum(d.get(c, 0.0) for d in copies) / len(copies) for c in names}
            out.append("| torch copy 256 MiB | " + " | ".join(f"{vals[c]:.6g}" for c in names) + " |")
            for c in ("FETCH_SIZE", "WRITE_SIZE"):
                if vals.get(c):
                    scale[c] = copy_kib * 1024 / vals[c]
        out.append("")
    if "FETCH_SIZE" in scale and "WRITE_SIZE" in scale:
        out.append(f"copy scale: FETCH_SIZE x {scale['FETCH_SIZE']:.1f} B, "
                   f"WRITE_SIZE x {scale['WRITE_SIZE']:.1f} B (256 MiB copy = 268435456 B each way)")
        for name, n, k, bias in shapes:
            c = per_shape.get(name, {})
            if "FETCH_SIZE" in c and "WRITE_SIZE" in c:
                rd = c["FETCH_SIZE"] * scale["FETCH_SIZE"]
                wr = c["WRITE_SIZE"] * scale["WRITE_SIZE"]
                alg = algorithmic_bytes(STEP_QTYPE, n, k, STEP_M, bias)
                out.append(f"traffic {name} {n}x{k}: {rd + wr:.0f} B per launch "
                           f"(read {rd:.0f}, write {wr:.0f}; algorithmic {alg}; "
                           f"ratio {(rd + wr) / alg:.3f})")
    print("\n".join(out))


TRAFFIC_SUMMARY = ROOT / "profiles" / "gemv_q5_0_m2_8b_step_counters.md"


def committed_traffic(name, n, k):
    """HBM bytes per launch of one step shape, read from the committed
    FETCH_SIZE / WRITE_SIZE summary (the "traffic" lines `--summarize` writes),
    or None when that summary is absent."""
    if not TRAFFIC_SUMMARY.exists():
        return None
    tag = f"traffic {name} {n}x{k}: "
    for line in TRAFFIC_SUMMARY.read_text().splitlines():
        if line.startswith(tag):
            return int(line[len(tag):].split()[0])
    return None


TIMELINE_CASES = (  # (label, qtype, n, k, fusion)
    ("qkv 5632x4608 + LayerNorm", "Q5_0", 5632, 4608, "ln"),
    ("qkv 5632x4608", "Q5_0", 5632, 4608, "plain"),
    ("o_proj 4608x4608 + residual", "Q5_0", 4608, 4608, "res"),
    ("qkv 5632x4608 + LayerNorm", "Q4_0", 5632, 4608, "ln"),
    ("o_proj 4608x4608 + residual", "Q4_0", 4608, 4608, "res"),
    ("lm_head 49152x4608 + LayerNorm", "Q5_0", 49152, 4608, "ln"),
    ("lm_head 49152x4608", "Q5_0", 49152, 4608, "plain"),
    ("c_fc 18432x4608", "Q5_0", 18432, 4608, "plain"),
    ("lm_head 49152x4608", "Q4_0", 49152, 4608, "plain"),
)


def timeline(dev, launches=10):
    """Per-phase timeline of the streaming MFMA GEMV (M = 2) from the stamps
    of libsvq_timeline.so, next to a coalesced plain read of the same bytes:
    `launches` back-to-back launches (weights rotated) in one graph, stamps of
    the fifth; launch time = first entry to last end of a launch, gap = to the
    next launch's first entry. Phase columns: 0 / 50 / 90th percentile over the
    busy waves, us after the launch's first entry (the LayerNorm phases only
    for cases with a LayerNorm); the last column is the
    median end of the waves of the first and of the second half of the
    workgroups (with two workgroups per CU, the first half holds one per CU).
    Prints a markdown table."""
    lib = ctypes.CDLL(str(Path(native.__file__).resolve().parent / "libsvq_timeline.so"))
    vp, i32 = ctypes.c_void_p, ctypes.c_int
    lib.svq_gemv_fused.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, vp,
                                   ctypes.c_float, vp, i32, vp]
    lib.svq_gemv_fused.restype = i32
    lib.svq_gemv.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp]
    lib.svq_timeline_stamps.argtypes = [vp]
    lib.svq_timeline_read.argtypes = [vp, ctypes.c_uint64, i32, vp, vp, vp]
    lib.svq_last_error.restype = ctypes.c_char_p
    stream = torch.cuda.Stream(dev)
    m, groups_read = 2, 512
    slots = 12  # per wave, as the timeline build writes them
    stamps = torch.zeros((launches, 4096 * 4 * slots), dtype=torch.int64, device=dev)
    sink = torch.empty(4096 * 256, dtype=torch.int32, device=dev)
    pool = Pool(dev, 1600 * 2**20, 160 * 2**20)

    def run(calls):
        g = capture(calls, stream)
        for _ in range(3):
            stamps.zero_()
            torch.cuda.synchronize()
            with torch.cuda.stream(stream):
                g.replay()
            stream.synchronize()
        return stamps.cpu().numpy().reshape(launches, -1, slots)

    def summary(st, phases, ln=False):
        first = [w[w[:, 0] > 0][:, 0].min() for w in st]
        last = [w[w[:, 0] > 0][:, 4].max() for w in st]
        dur = statistics.median((last[i] - first[i]) / 100 for i in range(1, launches - 1))
        gap = statistics.median((first[i + 1] - last[i]) / 100 for i in range(1, launches - 1))
        w = st[4][st[4][:, 0] > 0]
        t0 = w[:, 0].min()
        busy = w[w[:, 5] > 0] if phases else w
        pct = lambda c: "/".join(f"{v:.2f}" for v in np.percentile((busy[:, c] - t0) / 100,
                                                                   [0, 50, 90]))
        lns = [pct(c) for c in (8, 9, 10)] if ln else ["", "", ""]
        cols = ([pct(6), *lns] + [pct(c) for c in (1, 2, 3)]) if phases else [""] * 7
        ends = (st[4][:, 4] - t0) / 100
        live = st[4][:, 0] > 0
        half = np.arange(len(ends)) // 4 < live.sum() // 8  # workgroups of 4 waves
        split = "/".join(f"{np.median(ends[live & sel]):.2f}" for sel in (half, ~half))
        return [f"{dur:.2f}", f"{gap:.2f}", *cols, pct(4), split]

    print("| case | qtype | launch us | gap us | x issued | LN mean | LN variance | LN normalized "
          "| x staged | step 1 | tile 1 | end | end by half |")
    print("|---|---|---|---|---|---|---|---|---|---|---|---|---|")
    for label, qtype, n, k, fusion in TIMELINE_CASES:
        pool.reset()
        cps = pool.copies(qtype, n, k, launches)
        x = torch.randn((m, k), device=dev).half()
        y = torch.empty((m, n), device=dev, dtype=torch.half)
        res = torch.randn((m, n), device=dev).half()
        lw = (torch.rand(k, device=dev) + 0.5).half()
        lb = (torch.randn(k, device=dev) * 0.1).half()
        code = native.QTYPE_CODE[qtype]

        def gemv(i):
            q, sc = cps[i]
            lib.svq_timeline_stamps(stamps[i].data_ptr())
            if fusion == "plain":
                rc = lib.svq_gemv(x.data_ptr(), q.data_ptr(), sc.data_ptr(), None, y.data_ptr(),
                                  m, n, k, code, 0, stream.cuda_stream)
            else:
                ln = fusion == "ln"
                rc = lib.svq_gemv_fused(x.data_ptr(), q.data_ptr(), sc.data_ptr(), None,
                                        y.data_ptr(), m, n, k, code,
                                        lw.data_ptr() if ln else None,
                                        lb.data_ptr() if ln else None, 1e-5,
                                        None if ln else res.data_ptr(), 0, stream.cuda_stream)
            lib.svq_timeline_stamps(None)
            if rc:
                raise RuntimeError(lib.svq_last_error().decode())

        print(f"| {label} | {qtype} | " + " | ".join(summary(run([lambda i=i: gemv(i) for i in
                                                                  range(launches)]), True,
                                                             fusion == "ln")) + " |")
        nbytes = (cps[0][0].numel() + cps[0][1].numel() * 2) // 1024 * 1024

        def read(i):
            rc = lib.svq_timeline_read(cps[i][0].data_ptr(), nbytes, groups_read, sink.data_ptr(),
                                       stamps[i].data_ptr(), stream.cuda_stream)
            if rc:
                raise RuntimeError(lib.svq_last_error().decode())

        print(f"| plain read, {nbytes / 1e6:.1f} MB | | " +
              " | ".join(summary(run([lambda i=i: read(i) for i in range(launches)]), False)) + " |")
        sys.stdout.flush()


def host_cores():
    """(threads the CPU baselines use, the host's CPU count): every CPU this
    process may run on (its affinity mask, which on a GPU box is the share
    of the host its job is given), and os.cpu_count() for the record."""
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    return usable, os.cpu_count()


def cpu_baseline():
    """The reference's CPU path (tiled fp32 dequantize + F.linear), restated
    in oracle/, for one pass of the step at batch 2, timed on this host."""
    from oracle import soa_oracle as orc
    threads, host_cpus = host_cores()
    torch.set_num_threads(threads)
    total_bytes, elapsed = 0, 0.0
    per = []
    for name, n, k, bias in STEP_SHAPES:
        q, s = orc.synthetic_soa(STEP_QTYPE, n, k, seed=n)
        qt, st = torch.from_numpy(q), torch.from_numpy(s)
        x = torch.randn(STEP_M, k)
        b = torch.randn(n) if bias else None
        orc.tiled_linear_cpu(x, qt, st, STEP_QTYPE, n, k, b)  # warm-up
        runs = []
        for _ in range(3):
            t0 = time.perf_counter()
            orc.tiled_linear_cpu(x, qt, st, STEP_QTYPE, n, k, b)
            runs.append(time.perf_counter() - t0)
        t = statistics.median(runs)
        per.append({"shape": f"{name} {n}x{k}", "ms": round(t * 1e3, 2)})
        total_bytes += algorithmic_bytes(STEP_QTYPE, n, k, STEP_M, bias)
        elapsed += t
    return {"value": round(total_bytes / elapsed / 1e9, 2), "unit": "GB/s", "cores": threads,
            "host_cpus": host_cpus, "kind": "port",
            "sample": "one pass of the Q5_0 batch-2 8B step (5 GEMVs) through the reference's "
                      "CPU path (tiled fp32 dequantize + F.linear), median of 3",
            "ms_per_step": round(elapsed * 1e3, 1), "per_shape": per}


def cpu_sweep():
    """Every `sweep` configuration (configs 1-4) through the reference's CPU
    path on the host cores: ms per GEMV (median of 3 after one warm-up) and
    GB/s of algorithmic bytes."""
    from oracle import soa_oracle as orc
    threads, host_cpus = host_cores()
    torch.set_num_threads(threads)
    rows, mats = [], {}
    for cfg_name, qtype, n, k, m, bias in sweep_cases():
        if (qtype, n, k) not in mats:
            mats.clear()  # one matrix resident at a time (cases are grouped by shape)
            q, s = orc.synthetic_soa(qtype, n, k, seed=n + k)
            mats[qtype, n, k] = (torch.from_numpy(q), torch.from_numpy(s))
        qt, st = mats[qtype, n, k]
        gen = torch.Generator().manual_seed(m)
        x = torch.randn((m, k), generator=gen)
        b = torch.randn(n, generator=gen) if bias else None
        orc.tiled_linear_cpu(x, qt, st, qtype, n, k, b)
        runs = []
        for _ in range(3):
            t0 = time.perf_counter()
            orc.tiled_linear_cpu(x, qt, st, qtype, n, k, b)
            runs.append(time.perf_counter() - t0)
        t = statistics.median(runs)
        nbytes = algorithmic_bytes(qtype, n, k, m, bias)
        rows.append({"config": cfg_name, "qtype": qtype, "n": n, "k": k, "m": m,
                     "ms": round(t * 1e3, 3), "gbs": round(nbytes / t / 1e9, 3)})
    return {"cores": threads, "host_cpus": host_cpus, "kind": "port",
            "sample": "each sweep configuration once through the reference's CPU path (tiled "
                      "fp32 dequantize + F.linear), median of 3 after a warm-up",
            "cases": rows}


# Decode loops. StarCoder2-8B-style: 32 layers, Q4_0 weights, beam 2, a
# 1024-token prefill whose first 576 vectors are the seeded vision prompt
# (SigLIP's 576 image tokens), then a fixed number of decode steps (random
# end-of-sequence tokens cannot stop it). GPTBigCode-1B: 24 layers, Q4_0
# linears with Q8_0 token / position tables (as the reference's converter
# writes Q4_0 files), the same loop with a 257-vector vision prompt (CLIP's
# 257 image tokens).
DECODE = {"qtype": "Q4_0", "beams": 2, "prompt": 576, "prefill": 1024, "steps": 512}
DECODE_1B = {"qtype": "Q4_0", "embed_qtype": "Q8_0", "beams": 2, "prompt": 257, "prefill": 1024,
             "steps": 512}


def decode_model(dev, family="8b"):
    from starvector_amd.decoder import (BigCodeConfig, DecoderConfig, GPTBigCodeDecoder,
                                        Starcoder2Decoder)
    if family == "8b":
        cfg = DecoderConfig()
        return cfg, Starcoder2Decoder(cfg, qtype=DECODE["qtype"], seed=0, device=dev)
    cfg = BigCodeConfig()
    return cfg, GPTBigCodeDecoder(cfg, qtype=DECODE_1B["qtype"],
                                  embed_qtype=DECODE_1B["embed_qtype"], seed=0, device=dev)


def decode_prompt(cfg, dev, length, vision, dtype=torch.float16):
    """The seeded vision prompt (`vision` fp16 N(0,1) vectors), extended with
    further seeded vectors to `length` prefill tokens."""
    g = torch.Generator(device=dev).manual_seed(1)
    head = torch.randn((1, min(length, vision), cfg.hidden), generator=g, device=dev)
    extra = torch.randn((1, max(0, length - vision), cfg.hidden), generator=g, device=dev)
    return torch.cat((head, extra), 1).to(dtype)


def run_decode(model, emb, steps, sync, beams, as_specified=False):
    """Beam decode of `steps` steps; returns wall-clock marks (seconds). As
    specified: the reference's loop (whole-vocabulary torch warpers,
    torch.multinomial, host survivor selection) over the decoder's torch
    attention / LayerNorm path; otherwise the fused loop."""
    from starvector_amd.decoder import beam_steps, beam_steps_reference
    marks = {}

    def mark(key):
        sync()
        marks[key] = time.perf_counter()

    loop = beam_steps_reference if as_specified else beam_steps
    model.fused = not as_specified
    torch.manual_seed(0)
    with torch.inference_mode():
        mark("start")
        loop(model, emb, steps, beams, on_prefill=lambda: mark("prefill"),
             on_step=lambda i: mark("first") if i == 1 else None)
        mark("end")
    return marks


def decode_bench(dev, steps, family="8b"):
    """Decode rates of one decoder on the GPU, as specified and fused."""
    spec = DECODE if family == "8b" else DECODE_1B
    cfg, model = decode_model(dev, family)
    sync = torch.cuda.synchronize
    out = {"workload": decode_workload(cfg, spec, family, steps), "steps": steps,
           "weight_bytes_per_step": decoder_weight_bytes(cfg, spec)}
    for mode in ("as_specified", "fused"):
        as_specified = mode == "as_specified"
        # Warm-up: loads kernels and GEMM libraries.
        run_decode(model, decode_prompt(cfg, dev, 64, spec["prompt"]), 3, sync, spec["beams"],
                   as_specified)
        marks = run_decode(model, decode_prompt(cfg, dev, spec["prefill"], spec["prompt"]), steps,
                           sync, spec["beams"], as_specified)
        decode_s = marks["end"] - marks["first"]
        out[mode] = {
            "decode_steps_per_s": round((steps - 1) / decode_s, 2),
            "decode_ms_per_step": round(decode_s / (steps - 1) * 1e3, 3),
            "tokens_per_s_incl_prefill": round(steps / (marks["end"] - marks["start"]), 2),
            "prefill_ms": round((marks["prefill"] - marks["start"]) * 1e3, 1),
            "first_step_ms": round((marks["first"] - marks["prefill"]) * 1e3, 1),
            "ops": ("reference: HIP GEMV per quantized linear; torch LayerNorm, attention, GELU, "
                    "residual adds; whole-vocabulary torch warpers, torch.multinomial, host "
                    "survivor selection" if as_specified else
                    "fused: LayerNorm / GELU / residual inside the HIP GEMVs, HIP decode "
                    "attention, HIP beam candidates and selection"),
        }
    model.fused = True
    return out, model, cfg


def decode_workload(cfg, spec, family, steps):
    if family == "8b":
        arch = (f"StarCoder2-8B-style decoder, {cfg.layers} layers, hidden {cfg.hidden}, "
                f"{cfg.heads}/{cfg.kv_heads} heads, inner {cfg.inner}, vocab {cfg.vocab}, "
                f"{spec['qtype']} weights")
    else:
        arch = (f"GPTBigCode-1B decoder, {cfg.layers} layers, hidden {cfg.hidden}, {cfg.heads} "
                f"heads (multi-query), inner {cfg.inner}, vocab {cfg.vocab}, {spec['qtype']} "
                f"linears, {spec['embed_qtype']} token / position tables")
    return (f"{arch} (seeded synthetic), beam {spec['beams']}, prefill {spec['prefill']} tokens "
            f"({spec['prompt']}-vector vision prompt), {steps} decode steps")


def decoder_weight_bytes(cfg, spec):
    bb = BLOCK_BYTES[spec["qtype"]]
    if "embed_qtype" in spec:  # GPTBigCode: c_attn, attn c_proj, c_fc, mlp c_proj
        per_layer = [(cfg.hidden + 2 * cfg.head_dim, cfg.hidden), (cfg.hidden, cfg.hidden),
                     (cfg.inner, cfg.hidden), (cfg.hidden, cfg.inner)]
        head_bb = BLOCK_BYTES[spec["embed_qtype"]]
    else:
        per_layer = [(cfg.hidden + 2 * cfg.kv_heads * cfg.head_dim, cfg.hidden),
                     (cfg.hidden, cfg.hidden), (cfg.inner, cfg.hidden), (cfg.hidden, cfg.inner)]
        head_bb = bb
    return (cfg.layers * sum(n * k // 32 * bb for n, k in per_layer) +
            cfg.vocab * cfg.hidden // 32 * head_bb)


def decode_cpu_baseline(model, cfg, steps=2, prompt=16):
    """The same decoder on the host cores through the reference's CPU path
    (fp32; every quantized linear as tiled dequantize + F.linear) and the
    reference's loop, for a short prompt and a few decode steps."""
    threads, host_cpus = host_cores()
    torch.set_num_threads(threads)
    model.to_host()
    emb = decode_prompt(cfg, torch.device("cpu"), prompt, DECODE["prompt"], torch.float32)
    marks = run_decode(model, emb, steps, lambda: None, DECODE["beams"], as_specified=True)
    per_step = (marks["end"] - marks["prefill"]) / steps
    return {"decode_steps_per_s": round(1 / per_step, 4), "decode_ms_per_step": round(per_step * 1e3, 1),
            "cores": threads, "host_cpus": host_cpus, "kind": "port",
            "sample": f"{steps} beam-2 decode steps after a {prompt}-token prefill, same 32-layer "
                      f"model on the host in fp32 (reference CPU path per quantized linear)"}


def summarize_decode(trace: Path):
    """GEMV share of the decode steps in a kernel trace of `--decode-only`:
    dispatches after the last dequantize kernel of the measured prefill."""
    rows = sorted(_read_csv(trace), key=lambda r: int(r["Dispatch_Id"]))
    last = max(i for i, r in enumerate(rows) if "dequant_kernel" in r["Kernel_Name"])
    phase = rows[last + 1:]
    durs = _durations_us(phase)
    total = sum(durs)
    gemv = sum(d for d, r in zip(durs, phase)
               if _is_gemv(r["Kernel_Name"]) or _is_split_finish(r["Kernel_Name"]))
    by = {}
    for d, r in zip(durs, phase):
        key = _short_kernel(r["Kernel_Name"])[:70]
        t, n = by.get(key, (0.0, 0))
        by[key] = (t + d, n + 1)
    span = (int(phase[-1]["End_Timestamp"]) - int(phase[0]["Start_Timestamp"])) / 1e3
    out = [f"decode phase: {len(phase)} dispatches, kernel time {total:.0f} us, span {span:.0f} us",
           f"GEMV kernels: {gemv:.0f} us = {gemv / total:.1%} of kernel time, {gemv / span:.1%} of the span",
           "| kernel | calls | avg us | total us | share |", "|---|---|---|---|---|"]
    for key, (d, n) in sorted(by.items(), key=lambda kv: -kv[1][0])[:15]:
        out.append(f"| {key} | {n} | {d / n:.2f} | {d:.0f} | {d / total:.1%} |")
    print("\n".join(out))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--trials", type=int, default=5, help="timed trials of --steps steps each")
    ap.add_argument("--quick", action="store_true", help="skip the sweep and CPU baseline")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--summarize", metavar="DIR",
                    help="summarize rocprofv3 CSV output of --profile runs under DIR (kernel "
                         "trace and counter collections) per step GEMV shape, then exit")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode-loop measurement")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the decode loop (for kernel traces) and print its JSON")
    ap.add_argument("--decode-steps", type=int, default=DECODE["steps"])
    ap.add_argument("--decode-family", choices=("8b", "1b"), default="8b",
                    help="decoder of --decode-only")
    ap.add_argument("--summarize-decode", metavar="CSV",
                    help="GEMV share of the decode steps in a kernel trace of --decode-only, then exit")
    ap.add_argument("--timeline", action="store_true",
                    help="per-phase timeline of the GEMV (libsvq_timeline.so); prints a table")
    ap.add_argument("--profile", action="store_true",
                    help="eager launches for rocprofv3: every step GEMV on 8 copies, twice, then "
                         "16 torch copies of 256 MiB (the known-size copy that scales FETCH_SIZE "
                         "and WRITE_SIZE); prints nothing else")
    args = ap.parse_args()
    if args.summarize:
        summarize(Path(args.summarize))
        return
    if args.summarize_decode:
        summarize_decode(Path(args.summarize_decode))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the path runs on one GPU; see DESIGN.md for how it would shard)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU")
    dev = torch.device("cuda:0")
    native.load()
    stream = torch.cuda.Stream(dev)
    log(f"device: {torch.cuda.get_device_name(dev)}")
    if args.profile:
        profile_pass(dev, stream)
        return
    if args.timeline:
        timeline(dev)
        return
    if args.decode_only:
        result, _, _ = decode_bench(dev, args.decode_steps, args.decode_family)
        print(json.dumps(result), flush=True)
        return
    if args.steps < 1 or args.warmup < 0 or args.trials < 1:
        sys.exit("--steps and --trials must be positive, --warmup not negative")

    # --- headline step: 8 passes over the 5 matrices, distinct copies -------
    pool = Pool(dev, q_bytes=3 * 2**30, s_bytes=2**29)
    gen = torch.Generator(device=dev).manual_seed(0)
    calls, step_bytes, head = [], 0, None
    per_shape = {name: [] for name, *_ in STEP_SHAPES}
    xs = {k: torch.randn((STEP_M, k), device=dev, generator=gen).half() for k in (4608, 18432)}
    for name, n, k, bias in STEP_SHAPES:
        cps = pool.copies(STEP_QTYPE, n, k, COPIES)
        b = torch.randn(n, device=dev, generator=gen).half() if bias else None
        y = torch.empty((STEP_M, n), dtype=torch.float16, device=dev)
        per_shape[name] = [make_call(xs[k], q, s, y, STEP_QTYPE, b) for q, s in cps]
        step_bytes += algorithmic_bytes(STEP_QTYPE, n, k, STEP_M, bias)
    # Exactly W untimed steps, then trials of exactly K steps: step i runs the
    # five matrices on copy i % COPIES (the warm-up's steps come first).
    def steps_graph(first, count):
        return capture([per_shape[name][(first + i) % COPIES]
                        for i in range(count) for name, *_ in STEP_SHAPES], stream)

    if args.warmup:
        warm = steps_graph(0, args.warmup)
        time_graph(warm, stream, 1)
        del warm
    graph = steps_graph(args.warmup, args.steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    trial_ms = [time_graph(graph, stream, 1) for _ in range(args.trials)]
    wall = time.perf_counter() - t0
    steps = args.steps
    ms_step = statistics.median(trial_ms) / steps
    value = step_bytes / (ms_step * 1e-3) / 1e9
    log(f"step: {ms_step * 1e3:.1f} us/step, {value:.1f} GB/s ({value / PEAK_HBM_GBS:.1%} of 8 TB/s), "
        f"median of {args.trials} trials of {steps} steps (wall {wall:.3f} s)")
    del graph

    # --- dominant launch: lm_head, own graph over its 8 copies -------------
    hname, hn, hk, hbias = STEP_SHAPES[-1]
    head_plan = native.gemv_plan(STEP_M, hn, hk, STEP_QTYPE)
    hgraph = capture(per_shape[hname], stream)
    time_graph(hgraph, stream, 2)
    head_ms = statistics.median(time_graph(hgraph, stream, 5) / COPIES for _ in range(5))
    head_bytes = algorithmic_bytes(STEP_QTYPE, hn, hk, STEP_M, hbias)
    achieved = head_bytes / (head_ms * 1e-3) / 1e9
    del hgraph
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": committed_traffic(hname, hn, hk),
                "traffic_source": TRAFFIC_SUMMARY.name,
                "kernel": f"{KERNEL_NAMES[head_plan['kernel']]} {STEP_QTYPE} M={STEP_M} lm_head {hn}x{hk}",
                "launch": head_plan,
                "us_per_launch": round(head_ms * 1e3, 2), "bytes_per_launch": head_bytes}
    log(f"lm_head: {head_ms * 1e3:.2f} us, {achieved:.1f} GB/s")

    sweep = []
    if not args.quick:
        for cfg, qtype, n, k, m, bias in sweep_cases():
            r = gemv_case(pool, dev, stream, qtype, n, k, m, bias)
            r["config"] = cfg
            sweep.append(r)
            log(f"{cfg} {qtype} {n}x{k} M={m}: {r['us']:.2f} us {r['gbs']:.0f} GB/s ({r['frac']:.1%})")

    dequant = []
    if not args.quick:
        for qtype in ("Q4_0", "Q5_0", "Q8_0"):
            for out_dtype in (torch.float16, torch.float32):
                r = dequant_case(pool, dev, stream, qtype, out_dtype)
                dequant.append(r)
                log(f"dequant {qtype} -> {r['out']}: {r['us']:.2f} us {r['gbs']:.0f} GB/s")

    cpu = cpu_rows = None
    if not args.quick and not args.no_cpu:
        log("cpu baseline ...")
        cpu = cpu_baseline()
        log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} threads "
            f"({cpu['host_cpus']} host CPUs)")
        cpu_rows = cpu_sweep()
        log(f"cpu sweep: {len(cpu_rows['cases'])} configurations")

    decode = None
    if not args.quick and not args.no_decode:
        decode = {}
        for family in ("1b", "8b"):
            result, model, cfg = decode_bench(dev, args.decode_steps, family)
            for mode in ("as_specified", "fused"):
                r = result[mode]
                log(f"decode {family} {mode}: {r['decode_steps_per_s']} steps/s "
                    f"({r['decode_ms_per_step']} ms/step), {r['tokens_per_s_incl_prefill']} "
                    f"tokens/s incl. prefill")
            if family == "8b" and not args.no_cpu:
                result["cpu_baseline"] = decode_cpu_baseline(model, cfg)
                log(f"decode cpu baseline: {result['cpu_baseline']['decode_ms_per_step']} ms/step")
            decode["starcoder2_8b" if family == "8b" else "gptbigcode_1b"] = result
            del model
            torch.cuda.empty_cache()

    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded Q5_0 blocks: uniform codes, fp16 scales U[1e-3,2e-2]; fp16 x ~ N(0,1))",
        "config": {"workload": "Q5_0 GEMV sweep over the StarCoder2-8B decoder linears, batch 2 "
                               "(qkv 5632x4608, o_proj 4608x4608, c_fc 18432x4608, c_proj 4608x18432, "
                               "lm_head 49152x4608)",
                   "batch": STEP_M, "bytes_per_step": step_bytes,
                   "frac_of_peak": round(value / PEAK_HBM_GBS, 4), "weight_copies": COPIES,
                   "trials": args.trials,
                   "trial_ms_per_step": [round(t / steps, 5) for t in trial_ms]},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_sweep": cpu_rows,
        "decode": decode,
        "sweep": sweep,
        "dequant": dequant,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
