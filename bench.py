"""Benchmark of the MI355X HFusion backend on BASELINE.json's workloads.

A step is one launch of a fused HFusion group over one batch of synthetic,
seeded input already resident in HBM.  The headline `value` is the group of
BASELINE configs[1] (fused RMSNorm + dynamic per-token int8 quant,
x bf16 [8192, 4096]) in algorithmic HBM GB/s; every other configured group is
measured the same way and reported under "groups" (GB/s, or TOPS for the W8A8
contraction) with its roofline fraction.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME] [--no-cpu]
    python bench.py --vendor OUT   # each group vs its eager PyTorch equivalent
    python bench.py --ceilings OUT # HBM rates of PyTorch's own streaming kernels
"""
import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "ascendnpu-ir_amd"))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0   # dense int8 MFMA, MI355X
BF16_PEAK_TFLOPS = 2500.0
HEADLINE = "rmsnorm_quant"
ORDER = ["rmsnorm_quant", "vec_add", "safe_softmax", "argmax", "w8a8_dequant"]
# further groups on the hot path, measured the same way (not BASELINE configs):
# the bf16 contraction, W8A8 with B as [K, N], a transpose fused with a cast,
# the block-scaled fp8 contraction (hfusion.matmul_mx)
EXTRA = ["bf16_mmad", "w8a8_dequant_kn", "transpose_cast", "mx_fp8", "mx_fp8_exact", "mx_fp4"]
# bench names that are a product group compiled with options
VARIANTS = {"mx_fp8_exact": ("mx_fp8", "mx_exact=1"),
            # the other kernels of the RMSNorm pattern, for --only runs
            "rmsnorm_quant_rowprog": ("rmsnorm_quant", "rmsq_kernel=0"),
            "rmsnorm_quant_rmsn": ("rmsnorm_quant", "rmsn_kernel=1")}
FP8_PEAK_TFLOPS = 5000.0  # dense fp8 MFMA (the block-scaled form runs at the same rate)
FP4_PEAK_TFLOPS = 10100.0  # dense fp4 (and fp6) MFMA


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def generic_inputs(meta, dev, seed=7):
    """Seeded random arguments from a group's parameter list (outputs empty)."""
    import numpy as np
    import torch
    rng = np.random.default_rng(seed)
    out = []
    scaled = "e8m0" in meta.get("variant", "")
    for idx, p in enumerate(meta["params"]):
        shape, elem = tuple(p["shape"]), p["elem"]
        if elem in ("f8E4M3FN", "f8E5M2") and p["role"] == "in":
            # every finite code (NaN / inf codes moved to finite neighbours)
            v = rng.integers(0, 256, shape).astype(np.uint8)
            v[(v & 0x7F) == 0x7F if elem == "f8E4M3FN" else (v & 0x7C) == 0x7C] &= 0xF7 if elem == "f8E4M3FN" else 0xF3
            dt = torch.float8_e4m3fn if elem == "f8E4M3FN" else torch.float8_e5m2
            out.append(torch.from_numpy(v).view(dt).to(dev))
            continue
        if scaled and elem == "i8" and p["role"] == "in" and idx < 2:
            # fp4 operand bytes: every code is a number
            out.append(torch.from_numpy(rng.integers(0, 256, shape).astype(np.uint8)).view(torch.int8).to(dev))
            continue
        if scaled and elem == "i8" and p["role"] == "in":
            # e8m0 block scales around 2^0
            out.append(torch.from_numpy(rng.integers(120, 135, shape).astype(np.uint8)).view(torch.int8).to(dev))
            continue
        if p["role"] != "in":
            dt = {"i8": torch.int8, "bf16": torch.bfloat16, "f32": torch.float32, "i32": torch.int32}[elem]
            out.append(torch.empty(shape, dtype=dt, device=dev))
        elif elem == "i8":
            # int8 operands as in the W8A8 config: U[-127, 127]
            out.append(torch.from_numpy(rng.integers(-127, 128, shape, dtype=np.int8)).to(dev))
        elif elem == "bf16":
            out.append(torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(dev).to(torch.bfloat16))
        elif elem == "f32":
            out.append(torch.from_numpy(rng.uniform(0.001, 0.02, shape).astype(np.float32)).to(dev))
        else:
            raise KeyError(elem)
    return out


def device_inputs(name, dev):
    """Inputs and destination buffers for config `name`, on the device."""
    import numpy as np
    import torch

    import hfusion_mi355x as hf
    cfg = hf.groups.CONFIGS[name]["kw"]
    ins = hf.inputs.config_inputs(name, **cfg)

    def dev_t(a, bf16=False):
        t = torch.from_numpy(np.ascontiguousarray(a))
        if bf16:
            t = t.view(torch.bfloat16)
        return t.to(dev)

    if name == "vec_add":
        a, b = ins
        return [dev_t(a), dev_t(b), torch.empty_like(dev_t(a))], ins
    if name == "rmsnorm_quant":
        x, g = ins
        r, c = x.shape
        return [dev_t(x, True), dev_t(g, True), torch.empty((r, c), dtype=torch.int8, device=dev),
                torch.empty((r,), dtype=torch.float32, device=dev)], ins
    if name == "safe_softmax":
        x, = ins
        return [dev_t(x), torch.empty(x.shape, dtype=torch.bfloat16, device=dev)], ins
    if name == "argmax":
        x, = ins
        r = x.shape[0]
        return [dev_t(x), torch.empty((r,), dtype=torch.float32, device=dev),
                torch.empty((r,), dtype=torch.int32, device=dev)], ins
    if name == "w8a8_dequant":
        a, b, st, sc = ins
        return [dev_t(a), dev_t(b), dev_t(st), dev_t(sc),
                torch.empty((a.shape[0], b.shape[0]), dtype=torch.bfloat16, device=dev)], ins
    raise KeyError(name)


MALL_BYTES = 256 << 20   # MI355X Infinity Cache: rotate input sets so no launch hits it warm


def input_sets(dargs):
    """Copies of the arguments (inputs and destinations) so that consecutive
    launches touch disjoint buffers whose total exceeds the last-level cache."""
    per_set = sum(t.numel() * t.element_size() for t in dargs)
    n = max(2, min(16, -(-(3 * MALL_BYTES) // per_set)))
    sets = [dargs]
    for _ in range(n - 1):
        sets.append([t.clone() for t in dargs])
    return sets


def time_group(grp, sets, steps, warmup, min_warm_s=0.25):
    """Kernel time per launch (ms): K back-to-back launches between two HIP
    events on the stream they are launched on, total / K.

    Warmup: at least W launches and at least `min_warm_s` of back-to-back
    work.  After the host has been idle the MI355X's clocks take tens of
    milliseconds of load to come back up (measured: a 4096^3 W8A8 launch runs
    ~10 % slower over its first ~100 launches after a 0.2 s pause than after
    1000), so a fixed handful of warmup launches would time the ramp, not the
    kernel.

    Timed region: the host must never leave the GPU idle between the K
    launches.  When one launch runs longer than the host takes to enqueue it,
    a lead of untimed launches queued just before the start event keeps the
    GPU busy (at full clock) while the host enqueues the K timed ones;
    otherwise a spin kernel covers the enqueue (the clocks sink while it
    spins, so this is the fallback: a group's packed launch enqueues in a few
    microseconds, well under any of the configs' kernels)."""
    import torch
    stream = torch.cuda.current_stream()
    n = len(sets)
    # a group's launches are checked and packed once per input set, so that the
    # host enqueues each step in a few microseconds
    if hasattr(grp, "launcher"):
        fns = [grp.launcher(*s) for s in sets]
        grp = lambda *a, _f=fns: _f[a[0]]()
        sets = [(k,) for k in range(n)]
    torch.cuda.synchronize()
    i = 0
    t0 = time.perf_counter()
    block_enq, block_wall = [], []
    while i < warmup or time.perf_counter() - t0 < min_warm_s:
        b0 = time.perf_counter()
        for _ in range(32):
            grp(*sets[i % n])
            i += 1
        b1 = time.perf_counter()
        torch.cuda.synchronize()
        b2 = time.perf_counter()
        block_enq.append((b1 - b0) / 32)
        block_wall.append((b2 - b0) / 32)
    enq = sorted(block_enq)[len(block_enq) // 2]      # host seconds per launch
    per = sorted(block_wall)[len(block_wall) // 2]    # >= GPU seconds per launch
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if per > 1.5 * enq:
        lead = int(2.0 * enq * steps / per) + 16
        for _ in range(lead):
            grp(*sets[i % n])
            i += 1
    else:
        cal0, cal1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        cal0.record(stream)
        torch.cuda._sleep(1 << 20)
        cal1.record(stream)
        torch.cuda.synchronize()
        s_per_cycle = cal0.elapsed_time(cal1) * 1e-3 / (1 << 20)
        torch.cuda._sleep(int(min(2.0, 2.0 * enq * steps + 0.005) / s_per_cycle))
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        grp(*sets[i % n])
        i += 1
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end), wall


def cpu_baseline(name, ins, budget_s=12.0):
    """The oracle's op-by-op C restatement of the reference CPU lowering, on
    one host core, over a bounded sample of the same workload."""
    import ctypes

    import numpy as np
    sys.path.insert(0, REPO)
    from oracle.interp import lib, ptr
    L = lib()
    if name == "rmsnorm_quant":
        x, g = ins
        rows = 1024
        xs = np.ascontiguousarray(x[:rows])
        q = np.empty((rows, x.shape[1]), np.int8)
        s = np.empty(rows, np.float32)
        fn = lambda: L.hfref_rmsnorm_quant(ptr(xs), ptr(g), ctypes.c_float(1e-6), ptr(q), ptr(s), rows, x.shape[1])
        nbytes = xs.nbytes + g.nbytes + q.nbytes + s.nbytes
        sample = f"{rows} of 8192 rows x 4096"
    elif name == "vec_add":
        a, b = ins
        o = np.empty_like(a)
        fn = lambda: L.hfref_vecadd_f32(ptr(a), ptr(b), ptr(o), a.size)
        nbytes = 3 * a.nbytes
        sample = "full 2^24 elements"
    elif name == "safe_softmax":
        x, = ins
        rows = 128
        xs = np.ascontiguousarray(x[:rows])
        o = np.empty(xs.shape, np.uint16)
        fn = lambda: L.hfref_softmax_bf16(ptr(xs), ptr(o), rows, x.shape[1])
        nbytes = xs.nbytes + o.nbytes
        sample = f"{rows} of 4096 rows x 32768"
    elif name == "argmax":
        x, = ins
        rows = 64
        xs = np.ascontiguousarray(x[:rows])
        v = np.empty(rows, np.float32)
        i = np.empty(rows, np.int32)
        fn = lambda: L.hfref_argmax(ptr(xs), ptr(v), ptr(i), rows, x.shape[1])
        nbytes = xs.nbytes + v.nbytes + i.nbytes
        sample = f"{rows} of 256 rows x 152064"
    elif name == "w8a8_dequant":
        a, b, st, sc = ins
        rows = 2
        o = np.empty((rows, b.shape[0]), np.uint16)
        fn = lambda: L.hfref_w8a8_dequant_rows(ptr(a), ptr(b), ptr(st), ptr(sc), ptr(o), a.shape[0], b.shape[0],
                                               a.shape[1], 0, rows)
        ops = 2.0 * rows * b.shape[0] * a.shape[1]
        sample = f"{rows} of 4096 rows (N=K=4096)"
    else:
        raise KeyError(name)
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    if name == "w8a8_dequant":
        return {"value": ops / med / 1e12, "unit": "TOPS", "cores": 1, "kind": "port",
                "sample": sample + f", median of {len(times)} runs"}
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": sample + f", median of {len(times)} runs"}


def cpu_baseline_mt(name, ins, budget_s=10.0):
    """The same C restatement run row-parallel on the host's cores (the
    reference CPU runner is single-threaded; this is the secondary figure):
    the full workload split into one row slice per thread, the C calls
    releasing the GIL.  Headline group only."""
    import ctypes
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    sys.path.insert(0, REPO)
    from oracle.interp import lib, ptr
    if name != "rmsnorm_quant":
        return None
    L = lib()
    x, g = ins
    rows, cols = x.shape
    threads = max(1, min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()))
    xs = np.ascontiguousarray(x)
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    step = -(-rows // threads)

    def part(t):
        r0, r1 = t * step, min(rows, (t + 1) * step)
        if r0 < r1:
            L.hfref_rmsnorm_quant(ptr(xs[r0:]), ptr(g), ctypes.c_float(1e-6), ptr(q[r0:]), ptr(s[r0:]), r1 - r0, cols)
    nbytes = xs.nbytes + g.nbytes + q.nbytes + s.nbytes
    times = []
    with ThreadPoolExecutor(threads) as ex:
        t_end = time.perf_counter() + budget_s
        while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 20):
            t0 = time.perf_counter()
            list(ex.map(part, range(threads)))
            times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"all {rows} rows x {cols}, {threads} row slices in parallel, median of {len(times)} runs"}


def _csv_rows(d, suffix):
    import csv
    import glob
    rows = []
    for f in sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True)):
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    if not rows:
        raise SystemExit(f"no *{suffix} under {d}")
    return rows


def summarize_stats(d, out, command):
    """Text summary of a `rocprofv3 --kernel-trace --stats --output-format csv` run."""
    rows = [r for r in _csv_rows(d, "_kernel_stats.csv") if r["Name"].startswith("hf_")]
    with open(out, "w") as fh:
        fh.write(f"# rocprofv3 kernel statistics (MI355X, one GPU)\n# command: {command}\n")
        fh.write(f"{'kernel':32s} {'calls':>6s} {'avg_us':>10s} {'min_us':>10s} {'max_us':>10s}\n")
        for r in rows:
            fh.write(f"{r['Name']:32s} {int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:10.2f} "
                     f"{float(r['MinNs']) / 1e3:10.2f} {float(r['MaxNs']) / 1e3:10.2f}\n")


# bytes the calibration kernel (hf_vec_add, f32 [2^24]: two reads, one write)
# moves per launch; FETCH_SIZE / WRITE_SIZE of the same launch give the scale
# from counter KiB to HBM bytes
CALIB_KERNEL = "hf_vec_add"
CALIB_READ, CALIB_WRITE = 2 * 4 * (1 << 24), 4 * (1 << 24)


def summarize_pmc(fetch_dir, write_dir, out, command):
    """HBM traffic per launch from two `rocprofv3 --pmc` passes (FETCH_SIZE,
    WRITE_SIZE; KiB per dispatch), each scaled by what the counter reads for
    the calibration kernel of known size."""
    def per_kernel(d, counter):
        acc = {}
        for r in _csv_rows(d, "_counter_collection.csv"):
            if r["Counter_Name"] != counter or not r["Kernel_Name"].startswith("hf_"):
                continue
            acc.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        return {k: statistics.median(v) for k, v in acc.items()}
    fetch, write = per_kernel(fetch_dir, "FETCH_SIZE"), per_kernel(write_dir, "WRITE_SIZE")
    ff = CALIB_READ / (fetch[CALIB_KERNEL] * 1024.0)
    fw = CALIB_WRITE / (write[CALIB_KERNEL] * 1024.0)
    with open(out, "w") as fh:
        fh.write(f"# HBM traffic per launch from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (MI355X)\n"
                 f"# command: {command}\n"
                 f"# calibration: {CALIB_KERNEL} moves {CALIB_READ} B read + {CALIB_WRITE} B written per launch;\n"
                 f"#   FETCH_SIZE factor {ff:.4f}, WRITE_SIZE factor {fw:.4f} (bytes per counter byte)\n")
        for k in sorted(set(fetch) & set(write)):
            tb = fetch[k] * 1024.0 * ff + write[k] * 1024.0 * fw
            fh.write(f"traffic {k} fetch_kib={fetch[k]:.1f} write_kib={write[k]:.1f} bytes={tb:.0f}\n")


def summarize_counters(d, out, command):
    """Median per dispatch of every counter of one `rocprofv3 --pmc` csv run,
    per hf_ kernel.  SQ_INSTS_VALU_MFMA_MOPS_I8 counts int8 matrix operations
    in units of 512; SQ_VALU_MFMA_BUSY_CYCLES is summed over the 1024 SIMDs
    (256 CUs x 4), so / 1024 gives the busy cycles of one SIMD; SQ_BUSY_CYCLES
    is summed over the 32 shader engines (8 XCDs x 4)."""
    acc = {}
    for r in _csv_rows(d, "_counter_collection.csv"):
        if r["Kernel_Name"].startswith("hf_"):
            acc.setdefault(r["Kernel_Name"], {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    with open(out, "w") as fh:
        fh.write(f"# rocprofv3 --pmc counters per dispatch, median over dispatches (MI355X)\n# command: {command}\n")
        for k in sorted(acc):
            med = {c: statistics.median(v) for c, v in acc[k].items()}
            fh.write(f"{k}: " + " ".join(f"{c}={v:.0f}" for c, v in sorted(med.items())) + "\n")
            if "SQ_INSTS_VALU_MFMA_MOPS_I8" in med:
                fh.write(f"  int8 matrix ops = {med['SQ_INSTS_VALU_MFMA_MOPS_I8'] * 512:.4e}\n")
            if "SQ_INSTS_VALU_MFMA_MOPS_F8" in med:
                fh.write(f"  fp8 matrix flops = {med['SQ_INSTS_VALU_MFMA_MOPS_F8'] * 512:.4e}\n")
            if "SQ_VALU_MFMA_BUSY_CYCLES" in med and "GRBM_GUI_ACTIVE" in med:
                fh.write(f"  MFMA busy / GPU active cycles (GRBM_GUI_ACTIVE / 8 XCDs) = "
                         f"{med['SQ_VALU_MFMA_BUSY_CYCLES'] / 1024 / (med['GRBM_GUI_ACTIVE'] / 8):.3f}\n")
            if "SQ_WAIT_INST_LDS" in med and "SQ_WAVE_CYCLES" in med:
                fh.write(f"  wave cycles waiting on LDS instructions / wave cycles = "
                         f"{med['SQ_WAIT_INST_LDS'] / max(1.0, med['SQ_WAVE_CYCLES']):.3f}\n")
            if "SQ_VALU_MFMA_BUSY_CYCLES" in med:
                fh.write(f"  MFMA busy cycles per SIMD = {med['SQ_VALU_MFMA_BUSY_CYCLES'] / 1024:.0f}\n")
            if "SQ_BUSY_CYCLES" in med:
                fh.write(f"  SQ busy cycles per shader engine (/ 32 SEs) = {med['SQ_BUSY_CYCLES'] / 32:.0f}\n")
            if "SQ_LDS_IDX_ACTIVE" in med and "SQ_LDS_BANK_CONFLICT" in med:
                fh.write(f"  LDS bank-conflict cycles / LDS active cycles = "
                         f"{med['SQ_LDS_BANK_CONFLICT'] / max(1.0, med['SQ_LDS_IDX_ACTIVE']):.3f}\n")


def vendor_equivalent(name):
    """The same group written as eager PyTorch on ROCm (hipBLASLt for the int8
    GEMM, PyTorch's own reduction kernels otherwise), over the same device
    arguments.  A reported comparison only: its outputs are not checked
    against the oracle, and nothing in the product calls it."""
    import torch

    if name == "vec_add":
        return lambda a, b, o: torch.add(a, b, out=o)
    if name == "rmsnorm_quant":
        def f(x, g, q, s):
            xf = x.float()
            r = torch.rsqrt((xf * xf).mean(-1, keepdim=True) + 1e-6)
            y = xf * r * g.float()
            sc = y.abs().amax(-1, keepdim=True) / 127.0
            q.copy_(torch.round(y / sc).clamp_(-127, 127).to(torch.int8))
            s.copy_(sc.squeeze(-1))
        return f
    if name == "safe_softmax":
        return lambda x, o: o.copy_(torch.softmax(x, -1))
    if name == "argmax":
        def f(x, v, i):
            mv, mi = torch.max(x, -1)
            v.copy_(mv)
            i.copy_(mi)
        return f
    if name == "w8a8_dequant":
        def f(a, b, st, sc, o):
            c = torch._int_mm(a, b.t())
            o.copy_(c.float() * st[:, None] * sc[None, :])
        return f
    raise KeyError(name)


def vendor_report(out, steps, warmup, command):
    """Kernel time of each fused group next to its eager PyTorch equivalent
    (and, for W8A8, hipBLASLt's int8 GEMM alone), same inputs, same timing
    method; written as a text table."""
    import torch

    import hfusion_mi355x as hf
    dev = torch.device("cuda:0")
    lines = ["# fused group (this backend) vs the same group in eager PyTorch on ROCm, MI355X",
             f"# command: {command}" if command else "# command: python bench.py --vendor OUT",
             "# group            ours_us  eager_us  speedup"]
    for name in ORDER:
        log(f"[bench] vendor comparison: {name}")
        grp = hf.compile(hf.catalog.get(name), require_cached=True).load()
        dargs, _ = device_inputs(name, dev)
        sets = input_sets(dargs)
        ours = time_group(grp, sets, steps, warmup)[0] / steps * 1e3
        eager = time_group(vendor_equivalent(name), sets, steps, warmup)[0] / steps * 1e3
        lines.append(f"{name:18s} {ours:8.2f} {eager:9.2f} {eager / ours:8.2f}x")
        if name == "w8a8_dequant":
            gemm = time_group(lambda a, b, st, sc, o: torch._int_mm(a, b.t()), sets, steps, warmup)[0] / steps * 1e3
            ops = grp.meta["algo_ops"]
            lines.append(f"  hipBLASLt int8 GEMM alone (torch._int_mm, int32 out): {gemm:.2f} us = "
                         f"{ops / (gemm * 1e-6) / 1e12:.0f} TOPS; fused W8A8 here: {ops / (ours * 1e-6) / 1e12:.0f} TOPS")
        del dargs, sets
        torch.cuda.empty_cache()
    # the block-scaled fp8 group next to hipBLASLt's fp8 GEMM with one scale
    # per tensor (torch._scaled_mm; torch has no e8m0 block-scale form here)
    log("[bench] vendor comparison: mx_fp8")
    grp = hf.compile(hf.catalog.get("mx_fp8"), require_cached=True).load()
    dargs = generic_inputs(grp.meta, dev)
    sets = input_sets(dargs)
    ours = time_group(grp, sets, steps, warmup)[0] / steps * 1e3
    ops = grp.meta["algo_ops"]
    one = torch.ones((), dtype=torch.float32, device=dev)
    bt = [[a, b.t().contiguous().t()] for a, b, _, _ in sets]   # B column-major, as _scaled_mm takes it
    try:
        vend = time_group(lambda a, b: torch._scaled_mm(a, b, scale_a=one, scale_b=one, out_dtype=torch.float32),
                          bt, steps, warmup)[0] / steps * 1e3
        lines.append(f"mx_fp8             {ours:8.2f}  (hipBLASLt fp8 GEMM, per-tensor scales, f32 out: {vend:.2f} us = "
                     f"{ops / (vend * 1e-6) / 1e12:.0f} TFLOP/s; block-scaled here: {ops / (ours * 1e-6) / 1e12:.0f} TFLOP/s)")
    except Exception as e:  # noqa: BLE001 - report what the platform lacks
        lines.append(f"mx_fp8             {ours:8.2f}  (torch._scaled_mm unavailable: {type(e).__name__})")
    del dargs, sets, bt
    torch.cuda.empty_cache()
    text = "\n".join(lines) + "\n"
    if out == "-":
        sys.stdout.write(text)
    else:
        with open(out, "w") as f:
            f.write(text)


def ceilings_report(out, steps, warmup, command):
    """The HBM rates PyTorch's own streaming kernels reach on this part (read
    only: sum; write only: fill; copy; a + b), over 512 MiB per launch, inputs
    rotated through the same number of buffer sets as the groups: what "peak"
    means in practice next to the nominal 8 TB/s."""
    import torch
    dev = torch.device("cuda:0")
    n = (512 << 20) // 4
    cases = [
        ("read (torch.sum, f32)", lambda a, o: torch.sum(a, dim=0, out=o), lambda: [torch.randn(n, device=dev), torch.empty((), device=dev)], n * 4),
        ("write (fill_, f32)", lambda a: a.fill_(1.5), lambda: [torch.empty(n, device=dev)], n * 4),
        ("copy (copy_, f32)", lambda a, b: b.copy_(a), lambda: [torch.randn(n // 2, device=dev), torch.empty(n // 2, device=dev)], n * 4),
        ("a + b (torch.add, f32)", lambda a, b, o: torch.add(a, b, out=o),
         lambda: [torch.randn(n // 3, device=dev), torch.randn(n // 3, device=dev), torch.empty(n // 3, device=dev)], (n // 3) * 12),
    ]
    lines = ["# HBM rates of PyTorch's own streaming kernels on one MI355X (nominal peak 8 TB/s)",
             f"# command: {command}" if command else "# command: python bench.py --ceilings OUT",
             "# case                       us/launch   TB/s   of 8 TB/s"]
    for name, fn, make, nbytes in cases:
        log(f"[bench] ceiling: {name}")
        sets = input_sets(make())
        us = time_group(fn, sets, steps, warmup)[0] / steps * 1e3
        lines.append(f"{name:28s} {us:9.2f} {nbytes / us / 1e6:6.2f}   {nbytes / us / 1e6 / 8:.3f}")
        del sets
        torch.cuda.empty_cache()
    text = "\n".join(lines) + "\n"
    if out == "-":
        sys.stdout.write(text)
    else:
        with open(out, "w") as f:
            f.write(text)


def traffic_table():
    f = os.path.join(REPO, "profiles", "hbm_traffic.txt")
    t = {}
    if os.path.exists(f):
        for line in open(f):
            if line.startswith("traffic "):
                parts = line.split()
                t[parts[1]] = float(parts[-1].split("=")[1])
    return t


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default=None, help="measure one group (e.g. for rocprofv3)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--warm-seconds", type=float, default=0.25,
                    help="minimum untimed back-to-back work before each group's timed steps (clock ramp)")
    ap.add_argument("--summarize-stats", nargs=2, metavar=("DIR", "OUT"),
                    help="write a text summary of a rocprofv3 --stats csv run")
    ap.add_argument("--summarize-pmc", nargs=3, metavar=("FETCH_DIR", "WRITE_DIR", "OUT"),
                    help="write the HBM traffic table from two rocprofv3 --pmc csv runs")
    ap.add_argument("--summarize-counters", nargs=2, metavar=("DIR", "OUT"),
                    help="write per-kernel medians of a rocprofv3 --pmc csv run")
    ap.add_argument("--command", default="", help="the profiling command, recorded in the summary")
    ap.add_argument("--vendor", metavar="OUT", default=None,
                    help="time each group against its eager PyTorch/hipBLASLt equivalent, write a table to OUT")
    ap.add_argument("--ceilings", metavar="OUT", default=None,
                    help="time PyTorch's own streaming kernels (read/write/copy/add), write a table to OUT")
    args = ap.parse_args()
    if args.ceilings:
        ceilings_report(args.ceilings, args.steps, args.warmup, args.command)
        return
    if args.summarize_stats:
        summarize_stats(*args.summarize_stats, args.command)
        return
    if args.summarize_counters:
        summarize_counters(*args.summarize_counters, args.command)
        return
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc, args.command)
        return
    if args.vendor:
        vendor_report(args.vendor, args.steps, args.warmup, args.command)
        return
    if args.gpus != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (each group shards by rows/columns "
              "with no exchange; see DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    import hfusion_mi355x as hf
    dev = torch.device("cuda:0")
    names = [args.only] if args.only else ORDER + EXTRA
    groups = {}
    headline_cpu = None
    headline_cpu_mt = None
    traffic = traffic_table()
    for name in names:
        log(f"[bench] {name}: preparing inputs")
        base, opts = VARIANTS.get(name, (name, ""))
        art = hf.compile(hf.catalog.get(base), options=opts, require_cached=True)
        grp = art.load()
        if name in EXTRA:
            dargs, host_ins = generic_inputs(grp.meta, dev), None
        else:
            dargs, host_ins = device_inputs(base, dev)
        log(f"[bench] {name}: timing {args.steps} steps")
        sets = input_sets(dargs)
        total_ms, wall = time_group(grp, sets, args.steps, args.warmup, args.warm_seconds)
        ms = total_ms / args.steps
        kern_ms = ms
        meta = grp.meta
        if meta["kind"] == "SINGLE_CUBE":
            ops = meta["algo_ops"]
            achieved = ops / (kern_ms * 1e-3) / 1e12
            bf16 = "bf16" in meta.get("variant", "")
            fp8 = "mfma_scale" in meta.get("variant", "")
            fp4 = fp8 and "e2m1" in meta.get("variant", "")
            peak, unit = ((BF16_PEAK_TFLOPS, "TFLOP/s") if bf16 else (FP4_PEAK_TFLOPS, "TFLOP/s") if fp4
                          else (FP8_PEAK_TFLOPS, "TFLOP/s") if fp8 else (INT8_PEAK_TOPS, "TOPS"))
            entry = {"value": ops * args.steps / (total_ms * 1e-3) / 1e12, "unit": unit, "ms_per_step": ms,
                     "roofline": {"bound": "mfma", "achieved": achieved, "peak": peak, "unit": unit,
                                  "frac": achieved / peak, "traffic": None}}
        else:
            nb = meta["algo_bytes"]
            achieved = nb / (kern_ms * 1e-3) / 1e9
            entry = {"value": nb * args.steps / (total_ms * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": ms,
                     "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                  "frac": achieved / HBM_PEAK_GBS, "traffic": None}}
        entry["roofline"]["traffic"] = traffic.get(meta["kernel"])
        entry["kernel"] = meta["kernel"]
        entry["algo_bytes"] = meta["algo_bytes"]
        entry["wall_s"] = wall
        groups[name] = entry
        log(f"[bench] {name}: {entry['value']:.1f} {entry['unit']} ({entry['roofline']['frac'] * 100:.1f}% of peak), "
            f"{ms * 1e3:.1f} us/step")
        if not args.no_cpu and host_ins is not None and (name == HEADLINE or args.only):
            log(f"[bench] {name}: CPU baseline (oracle restatement, 1 core)")
            headline_cpu = cpu_baseline(base, host_ins)
            headline_cpu_mt = cpu_baseline_mt(base, host_ins)
        entry["input_sets"] = len(sets)
        del dargs, sets
        torch.cuda.empty_cache()
    head = HEADLINE if HEADLINE in groups else names[0]
    head_base = VARIANTS.get(head, (head, ""))[0]
    h = groups[head]
    cfg = hf.groups.CONFIGS[head_base]["kw"] if head_base in hf.groups.CONFIGS else {}
    line = {
        "metric": "HBM GB/s (% of peak) per fused HFusion group; W8A8 mmad TOPS (% MFMA)",
        "value": h["value"], "unit": h["unit"], "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "warm_seconds": args.warm_seconds, "ms_per_step": h["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": {"rmsnorm_quant": "f32", "vec_add": "f32", "safe_softmax": "f32", "argmax": "f32",
                  "w8a8_dequant": "int8", "w8a8_dequant_kn": "int8", "bf16_mmad": "bf16",
                  "transpose_cast": "bf16", "mx_fp8": "fp8 (e4m3, e8m0 scales)",
                  "mx_fp8_exact": "fp8 (e4m3, e8m0 scales) via bf16", "mx_fp4": "fp4 (e2m1, e8m0 scales)"}[head_base if head_base != "mx_fp8" else head],
        "data": "synthetic (seeded splitmix64)",
        "config": {"workload": head, **{k: v for k, v in cfg.items()}},
        "roofline": h["roofline"],
        "cpu_baseline": headline_cpu,
        "cpu_baseline_mt": headline_cpu_mt,
        "groups": groups,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
