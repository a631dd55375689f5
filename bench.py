#!/usr/bin/env python3
"""Throughput of the fused CE + forward-KL distillation loss (fwd+bwd) on one
MI355X.

A step is one `distillation_loss` call over device-resident synthetic inputs:
logits GEMMs, fused row pass, grad_hidden and grad_W GEMMs, deferred mean,
INT8 round trip of grad_W, loss assembly. Default workload: Tied teacher,
BT=8192, H=4096, V=131072, bf16 inputs with fp32 accumulation, kd=0.4,
T=1.5, label smoothing 0.1, INT8 grad_W (16 chunks x 512 rows).

Prints one JSON line (see the repository's benchmark contract) with the
per-kernel roofline of the dominant kernel measured with HIP events on the
stream the kernels run on (in a second pass of the same number of steps, so
that the timed steps carry no events), and the CPU oracle timed on a bounded
sample.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "orda-cutile-rs_amd"))

PEAK_HBM_GBS = 8000.0           # MI355X HBM3E, GB/s
PEAK_MFMA_TFLOPS = {"bf16": 2500.0, "f32": 157.3}   # dense

WORKLOADS = {
    # name: (teacher, BT, H, Ht, V, dtype, kd, T, alpha, w_t, quant[, profile])
    "tied-8192x4096x131072-bf16-int8": ("tied", 8192, 4096, 4096, 131072, "bf16", 0.4, 1.5, 0.1,
                                        None, True),
    "tied-2048x4096x32000-f32": ("tied", 2048, 4096, 4096, 32000, "f32", 0.4, 1.5, 0.0, None,
                                 False),
    "separate-4096x2048x4096x32000-f32": ("separate", 4096, 2048, 4096, 32000, "f32", 0.5, 2.0,
                                          0.1, 1.0, False),
    "precomputed-4096x4096x65536-f32": ("precomputed", 4096, 4096, 4096, 65536, "f32", 0.7, 1.0,
                                        0.0, None, False),
    "tied-256x512x8192-f32": ("tied", 256, 512, 512, 8192, "f32", 0.4, 1.5, 0.0, None, False),
    # fp32 inputs under Profile::Fast (KernelConfig::fast_math: the row
    # pass's per-row logs and divisions approximate; the same fp32 pipeline)
    "tied-2048x4096x32000-f32-fast": ("tied", 2048, 4096, 4096, 32000, "f32", 0.4, 1.5, 0.0, None,
                                      False, "fast"),
    "separate-4096x2048x4096x32000-f32-fast": ("separate", 4096, 2048, 4096, 32000, "f32", 0.5,
                                               2.0, 0.1, 1.0, False, "fast"),
    "precomputed-4096x4096x65536-f32-fast": ("precomputed", 4096, 4096, 4096, 65536, "f32", 0.7,
                                             1.0, 0.0, None, False, "fast"),
    # the same Separate and Precomputed shapes with bf16 hidden rows and
    # weights (Precomputed logits stay fp32): the student's logits in bf16,
    # the teacher's fp32 logits read in the student logits GEMM's epilogue
    "separate-4096x2048x4096x32000-bf16": ("separate", 4096, 2048, 4096, 32000, "bf16", 0.5, 2.0,
                                           0.1, 1.0, False),
    "precomputed-4096x4096x65536-bf16": ("precomputed", 4096, 4096, 4096, 65536, "bf16", 0.7,
                                         1.0, 0.0, None, False),
    # wider decoders (H = 8192 and 16384, V = 128256) with the benchmark's
    # options, bf16 inputs, no INT8 step
    "tied-8192x8192x128256-bf16": ("tied", 8192, 8192, 8192, 128256, "bf16", 0.4, 1.5, 0.1, None,
                                   False),
    "tied-8192x16384x128256-bf16": ("tied", 8192, 16384, 16384, 128256, "bf16", 0.4, 1.5, 0.1,
                                    None, False),
}
DEFAULT = "tied-8192x4096x131072-bf16-int8"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_inputs(torch, wl, dev, seed=0):
    teacher, bt, h, ht, v, dt, *_ = wl
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32

    def normal(shape, std):
        x = torch.empty(shape, device=dev, dtype=torch.float32)
        x.normal_(0.0, std, generator=g)
        return x.to(tdt)
    s = normal((bt, h), 1.0)
    w = normal((v, h), 0.02)
    y = torch.randint(0, v, (bt,), device=dev, generator=g, dtype=torch.int64)
    if teacher == "tied":
        t = ("tied", normal((bt, h), 1.0))
    elif teacher == "separate":
        t = ("separate", normal((bt, ht), 1.0), normal((v, ht), 0.015))
    else:
        lg = torch.empty((bt, v), device=dev, dtype=torch.float32)
        lg.normal_(0.0, 2.0, generator=g)
        lg[torch.arange(bt, device=dev), y] += 8.0
        t = ("precomputed", lg)
    return s, w, y, t


def teacher_obj(H, t):
    if t[0] == "tied":
        return H.Teacher.Tied(t[1])
    if t[0] == "separate":
        return H.Teacher.Separate(t[1], t[2])
    return H.Teacher.Precomputed(t[1])


def profile_of(wl):
    return wl[11] if len(wl) > 11 else None


def compute_dtype(wl):
    """The dtype the GEMMs and logits run in: the inputs' own (Profile::Fast
    changes only the row pass's per-row logs and divisions)."""
    return wl[5]


def options(H, wl):
    _, _, _, _, _, _, kd, T, alpha, w_t, quant = wl[:11]
    cfg = H.KernelConfig(quantize_grad_weight=quant)
    if profile_of(wl) == "fast":
        cfg = H.KernelConfig.from_profile(H.Profile.Fast)
        cfg.quantize_grad_weight = quant
    return H.LossOptions(kd_weight=kd, temperature=T, label_smoothing=alpha,
                         teacher_ce_weight=w_t, config=cfg)


def work_per_step(wl, plan):
    """Algorithmic flops (GEMMs) and bytes (row pass, quant) of one step."""
    teacher, bt, h, ht, v, _, kd, T, alpha, w_t, quant = wl[:11]
    dt = compute_dtype(wl)
    es = 2 if dt == "bf16" else 4
    wt = w_t if w_t is not None else (1.0 if teacher == "tied" else 0.0)
    hs = h
    if teacher == "tied":
        fwd = 2 * (2 * bt) * h * v
        back_rows = 2 * bt if wt > 0 else bt
        dgrad = 2 * back_rows * v * h
        wgrad = 2 * back_rows * v * h
        t_rows_written = bt if wt > 0 else 0
    elif teacher == "separate":
        fwd = 2 * bt * v * (hs + ht)
        dgrad = 2 * bt * v * hs + (2 * bt * v * ht if wt > 0 else 0)
        wgrad = dgrad
        t_rows_written = bt if wt > 0 else 0
    else:
        fwd = 2 * bt * h * v
        dgrad = 2 * bt * v * h
        wgrad = dgrad
        t_rows_written = 0
    # row pass: read the student and teacher logits once, write the gradient
    # rows in the input dtype. Logits are stored in bf16 for bf16 inputs when
    # every loss term comes from the GEMM's fp32 accumulators (tied teacher,
    # or no KL term), else in fp32; with bf16 inputs, a KL term and a Separate
    # or Precomputed teacher, the student's in bf16 beside fp32 teacher
    # logits (read in the student logits GEMM's epilogue).
    rows_read = 2 * bt if (kd > 0 or wt > 0) else bt
    beside = dt == "bf16" and kd > 0 and teacher != "tied"
    ls = 2 if dt == "bf16" and (teacher == "tied" or kd == 0) else 4
    if beside:
        rowpass = bt * v * (2 + 4) + (bt + t_rows_written) * v * es
    else:
        rowpass = rows_read * v * ls + (bt + t_rows_written) * v * es
    # ... and, to form each row's lse at 1 and at T, the per-row statistics
    # the logits GEMM wrote: one 16-byte entry per 256-column tile (for
    # Precomputed teacher logits that the GEMM did not read, one per
    # 8192-column segment), the row pair's two 4-byte KL sums per tile where
    # the GEMM forms them, the label.
    nst = -(-v // 256)
    t_stats = (-(-v // 8192) if teacher == "precomputed" and not beside else nst) \
        if rows_read > bt else 0
    paired = dt == "bf16" and ((teacher == "tied" and (kd > 0 or wt > 0)) or beside)
    rowpass += bt * (nst * 16 + t_stats * 16 + (nst * 8 if paired else 0) + 8)
    # bf16 logits are stored relative to their 128-column half-tile maxima:
    # 4 bytes per half and row of the logits GEMM (Precomputed teacher rows
    # and fp32 teacher rows are stored as they are)
    if ls == 2 or beside:
        rowpass += bt * nst * 8 * (2 if rows_read > bt and teacher != "precomputed" and not beside
                                   else 1)
    quant_b = v * h * 8 if quant else 0
    return {"gemm_logits": ("mfma", fwd), "gemm_grad_hidden": ("mfma", dgrad),
            "gemm_grad_weight": ("mfma", wgrad), "row_pass": ("hbm", rowpass),
            "quant": ("hbm", quant_b)}


def cpu_info():
    """(model description, usable cores) of the host: the model name with the
    CPU family / model / stepping, clock and whether it runs under a
    hypervisor, as /proc/cpuinfo states them for the first processor."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if not line.strip():
                break
            k, _, val = line.partition(":")
            fields[k.strip()] = val.strip()
    except OSError:
        pass
    model = fields.get("model name", "unknown")
    extra = []
    if "cpu family" in fields:
        fam = fields["cpu family"]
        famx = f" (0x{int(fam):X})" if fam.isdigit() else ""
        extra.append(f"family {fam}{famx} model {fields.get('model', '?')} "
                     f"stepping {fields.get('stepping', '?')}")
    if "cpu MHz" in fields:
        extra.append(f"{float(fields['cpu MHz']):.0f} MHz")
    if "hypervisor" in fields.get("flags", "").split():
        extra.append("virtual machine")
    if extra:
        model = f"{model} ({', '.join(extra)})"
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    return model, cores


def cpu_baseline(wl, sample_rows=(2, 4, 6)):
    """The CPU oracle (one thread, as the reference: no threads, no
    dependencies) on a bounded sample of the same workload: one chunk of 2, 4
    and 6 rows (same H, V and options). A least-squares line through the three
    timings gives the cost per row and per chunk (the residual is reported);
    the per-call INT8 step is timed on its own so that it is not counted once
    per chunk. Extrapolated to the full BT in the Auto plan's chunks.

    The same measurement with the oracle's products, element-wise loops and
    INT8 rows shared out over the process's cores (OMP_NUM_THREADS at most;
    results bitwise the same) is reported beside it as `all_cores`."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as O
    import orda_hip as H
    teacher, bt, h, ht, v, dt, kd, T, alpha, w_t, quant = wl[:11]
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((v, h), dtype=np.float32) * 0.02).astype(np.float32)
    tw = (rng.standard_normal((v, ht), dtype=np.float32) * 0.015) if teacher == "separate" else None

    def mk(n):
        s = rng.standard_normal((n, h), dtype=np.float32)
        y = rng.integers(0, v, n)
        if teacher == "tied":
            t = H.Teacher.Tied(rng.standard_normal((n, h), dtype=np.float32))
        elif teacher == "separate":
            t = H.Teacher.Separate(rng.standard_normal((n, ht), dtype=np.float32), tw)
        else:
            t = H.Teacher.Precomputed(rng.standard_normal((n, v), dtype=np.float32) * 2)
        return s, y, t
    opts = options(H, wl)
    samples = [mk(n) for n in sample_rows]
    g = (rng.standard_normal((v, h), dtype=np.float32) * 1e-4).astype(np.float32) if quant else None
    plan = H.resolve_chunk_size(bt, H.ChunkSize.Auto, v, None)

    def measure(label):
        times = []
        for n, (s, y, t) in zip(sample_rows, samples):
            t0 = time.perf_counter()
            O.distillation_loss(s, w, y, t, opts)
            times.append(time.perf_counter() - t0)
            log(f"cpu oracle ({label}) sample BT={n}: {times[-1]:.2f} s")
        per_call = 0.0
        if quant:
            t0 = time.perf_counter()
            O.quant_dequant_grad_w(g, np.arange(8), -100)
            per_call = time.perf_counter() - t0
            log(f"cpu oracle ({label}) INT8 step alone: {per_call:.2f} s")
        x = np.array(sample_rows, np.float64)
        tt = np.array(times, np.float64)
        per_row, fixed = np.polyfit(x, tt, 1)
        per_row = max(float(per_row), 1e-9)
        resid = float(np.sqrt(np.mean((tt - (per_row * x + fixed)) ** 2)))
        per_chunk = max(float(fixed) - per_call, 0.0)
        est = bt * per_row + plan.num_chunks * per_chunk + per_call
        text = (f"one chunk of {', '.join(map(str, sample_rows))} rows of this workload "
                f"(same H, V, options; the reference's f32/f64 arithmetic), timed "
                f"{', '.join(f'{t:.2f}' for t in times)} s; least-squares per-row "
                f"{per_row:.3f} s and per-chunk {per_chunk:.3f} s (rms residual "
                f"{resid:.3f} s), per-call INT8 step {per_call:.2f} s timed alone; "
                f"extrapolated to BT={bt} in {plan.num_chunks} chunks ({est:.0f} s)")
        return bt / est, text

    model, cores = cpu_info()
    value, text = measure("one thread")
    out = {"value": value, "unit": "rows/s", "cores": 1, "kind": "port",
           "cpu": model, "host_cores": cores,
           "sample": f"oracle/liborda_oracle.so on one thread of a {cores}-core {model}: {text}"}
    try:
        threads = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))
    except ValueError:
        threads = cores
    if threads > 1:
        O.set_threads(threads)
        try:
            value_n, text_n = measure(f"{threads} threads")
        finally:
            O.set_threads(1)
        out["all_cores"] = {"value": value_n, "unit": "rows/s", "cores": threads,
                            "sample": (f"the same oracle with its products, element-wise loops "
                                       f"and INT8 rows shared out over {threads} threads "
                                       f"(results bitwise the same): {text_n}")}
    return out


def vendor_gemms(torch, wl, dev, s, w, t, reps):
    """The loss's three products on the same inputs' shapes, timed with the
    vendor library (hipBLASLt through torch: F.linear / torch.mm in the compute
    dtype, fp32 accumulation, output in the compute dtype, no fused epilogue),
    on this GPU in this run: a reference for what a tuned library reaches on
    these shapes here. Operands: the workload's hidden rows and weights, and a
    random gradient-like matrix (N(0, 1e-5^2)) in place of the row pass's
    output. Products as the library runs them: logits = hidden · Wᵀ,
    grad_hidden = dlogits · W, grad_W computed transposed = hiddenᵀ · dlogits.
    Separate teachers are not covered (two weights)."""
    import torch.nn.functional as F
    teacher, bt, h, ht, v, _, kd, T, alpha, w_t, quant = wl[:11]
    if teacher == "separate":
        return None
    dt = compute_dtype(wl)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    hid = s.to(tdt)
    if teacher == "tied" and (w_t is None or w_t > 0 or kd > 0):
        hid = torch.cat([hid, t[1].to(tdt)], 0)
    wt = w.to(tdt)
    rows = hid.shape[0]
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    dl = torch.empty((rows, v), device=dev, dtype=torch.float32)
    dl.normal_(0.0, 1e-5, generator=g)
    dl = dl.to(tdt)
    hid_t = hid.t().contiguous()
    products = {
        "gemm_logits": lambda: F.linear(hid, wt),
        # the plain product followed by one of the statistics the library's
        # logits epilogue forms (each row's logsumexp, one more pass over the
        # logits): a lower bound for the unfused form of that GEMM
        "gemm_logits_then_logsumexp": lambda: torch.logsumexp(F.linear(hid, wt), dim=1),
        "gemm_grad_hidden": lambda: torch.mm(dl, wt),
        "gemm_grad_weight": lambda: torch.mm(hid_t, dl),
    }
    flops = 2.0 * rows * h * v
    out = {"library": "hipBLASLt via torch (F.linear / torch.mm), "
                      f"{dt} in and out, fp32 accumulation, no fused epilogue",
           "peak_tflops": PEAK_MFMA_TFLOPS[dt]}
    for kind, fn in products.items():
        r = fn()
        torch.cuda.synchronize()
        del r
        times = []
        for _ in range(max(3, min(reps, 5))):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            r = fn()
            e1.record()
            e1.synchronize()
            times.append(e0.elapsed_time(e1))
            del r
        ms = sorted(times)[len(times) // 2]
        tf = flops / (ms * 1e-3) / 1e12
        out[kind] = {"ms": round(ms, 4), "achieved": round(tf, 2),
                     "frac": round(tf / PEAK_MFMA_TFLOPS[dt], 4)}
        log(f"vendor {kind}: {ms:.3f} ms ({tf:.1f} TFLOP/s)")
    del dl, hid, hid_t, wt
    return out


# ------------------------------------------------------------ profiles
KERNEL_CLASSES = (
    # (substring of the kernel name, kernel kind)
    ("gemm_kk_logits_", "gemm_logits"),
    ("gemm_kk_store_", "gemm_logits"),      # small fp32 problems: logits split over K
    ("gemm_kk_small_", "gemm_logits"),      # ... or on 128 x 128 tiles
    ("gemm_km_small_", "gemm_grad_hidden"),
    ("gemm_kmt_small_", "gemm_grad_weight"),
    ("gemm_km_", "gemm_grad_hidden"),
    ("gemm_kmt_", "gemm_grad_weight"),
    ("splitk_reduce", "splitk_reduce"),   # split-K: ordered sum of the partials
    ("transpose_rows", "transpose_rows"),   # grad_W's A operand: hidden rows transposed
    ("row_pass_", "row_pass"),            # row_pass_fused_kernel, row_pass_kernel
    ("row_consts_", "row_consts"),        # the chunked row pass: per-row constants ...
    ("row_grad_", "row_grad"),            # ... and the elementwise gradient
    ("row_kl_", "row_kl"),                # ... and, over fp32 logits, each row's KL
    ("row_stats_", "row_stats"),          # row_stats_kernel, row_stats_seg_kernel
    ("finalize_kernel", "finalize"),
    ("quant_", "quant"),                  # quant_vec_kernel, quant_kernel
    ("mark_targets", "mark_targets"),
    ("convert_rows", "convert_rows"),
)
COPY_KERNEL = "copyBuffer"          # HIP runtime's device-to-device copy kernel


def kernel_kind(name):
    for key, kind in KERNEL_CLASSES:
        if key in name:
            return kind
    if "copyBufferRect" in name:
        return "copy_rect"
    if COPY_KERNEL in name:
        return "copy"
    return None


def traffic_path(workload):
    return os.path.join(ROOT, "profiles", f"{workload.replace('-', '_')}_hbm_traffic.md")


def read_traffic(workload, kind):
    """HBM bytes per launch of `kind` from the committed PMC summary, or None."""
    import re
    path = traffic_path(workload)
    if not os.path.exists(path):
        return None
    m = re.search(r"^traffic-json: (\{.*\})$", open(path).read(), flags=re.M)
    if not m:
        return None
    rec = json.loads(m.group(1)).get(kind)
    return None if rec is None else rec["bytes_per_launch"]


def summarize(dirs, copy_bytes, timed_steps=0):
    """Markdown summary of rocprofv3 output directories: kernel-trace stats
    (per kernel kind) and, where present, FETCH_SIZE / WRITE_SIZE counter
    collections turned into HBM bytes per launch with the copy-kernel factor
    (bytes the copy moves / bytes the counter reports for it)."""
    import csv
    import glob
    from collections import defaultdict
    stats = defaultdict(lambda: [0, 0.0])           # kind -> [calls, total ns]
    counters = defaultdict(lambda: defaultdict(list))   # counter -> kind -> [value per dispatch]
    spans = defaultdict(dict)                       # kind -> {dispatch id: duration ns}
    trace = defaultdict(list)                       # kind -> [(start ns, duration ns)]
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                k = kernel_kind(r["Kernel_Name"])
                if k:
                    t0, t1 = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
                    trace[k].append((t0, t1 - t0))
        for f in glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                k = kernel_kind(r["Name"])
                if k:
                    stats[k][0] += int(r["Calls"])
                    stats[k][1] += float(r["TotalDurationNs"])
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                k = kernel_kind(r["Kernel_Name"])
                if k:
                    counters[r["Counter_Name"]][k].append(float(r["Counter_Value"]))
                    spans[k][r["Dispatch_Id"]] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    out = []
    if stats:
        # Steps are counted by the logits GEMM (one launch per group and step);
        # the timed-steps column averages each kind over its launches in the
        # last `timed_steps` steps, the steps bench.py times.
        steps = len(trace.get("gemm_logits", [])) or None
        hdr = "| kernel | calls | avg duration (ms) | total (ms) |"
        if timed_steps and steps:
            hdr += f" avg over the last {timed_steps} steps (ms) |"
        out.append(hdr)
        out.append("|---|---|---|---|" + ("---|" if timed_steps and steps else ""))
        for k, (n, ns) in sorted(stats.items(), key=lambda x: -x[1][1]):
            line = f"| {k} | {n} | {ns / n / 1e6:.4f} | {ns / 1e6:.3f} |"
            if timed_steps and steps:
                durs = [dt for _, dt in sorted(trace.get(k, []))]
                per_step = max(len(durs) // steps, 1)
                last = durs[-timed_steps * per_step:] if durs else []
                line += f" {sum(last) / len(last) / 1e6:.4f} |" if last else " - |"
            out.append(line)
    if "GRBM_GUI_ACTIVE" in counters and "SQ_VALU_MFMA_BUSY_CYCLES" in counters:
        # MI355X: 8 XCDs (GRBM_GUI_ACTIVE is summed over them) and 256 CUs x 4
        # SIMDs (the MFMA busy cycles are summed over the 1024 SIMDs).
        out.append("")
        out.append("| kernel | dispatches | duration (ms) | cycles per XCD | shader clock (GHz) | "
                   "MFMA busy cycles per SIMD | MFMA busy / elapsed cycles |")
        out.append("|---|---|---|---|---|---|---|")
        for k in sorted(counters["SQ_VALU_MFMA_BUSY_CYCLES"]):
            busy = counters["SQ_VALU_MFMA_BUSY_CYCLES"][k]
            grbm = counters["GRBM_GUI_ACTIVE"].get(k, [])
            if not grbm or max(busy) <= 0:
                continue
            n = len(grbm)
            cyc = sum(grbm) / n / 8
            dur = sum(spans[k].values()) / max(len(spans[k]), 1)
            simd = sum(busy) / len(busy) / 1024
            out.append(f"| {k} | {n} | {dur / 1e6:.3f} | {cyc:.4g} | {cyc / dur:.3f} | "
                       f"{simd:.4g} | {simd / cyc:.3f} |")
    traffic = {}
    if "FETCH_SIZE" in counters or "WRITE_SIZE" in counters:
        factors = {}
        for c in ("FETCH_SIZE", "WRITE_SIZE"):
            cp = counters.get(c, {}).get("copy")
            if cp and copy_bytes:
                factors[c] = copy_bytes / (max(cp) * 1024.0)
        out.append("")
        out.append("| kernel | FETCH_SIZE KiB/launch | WRITE_SIZE KiB/launch | "
                   "HBM bytes/launch (calibrated) |")
        out.append("|---|---|---|---|")
        kinds = sorted(set(counters.get("FETCH_SIZE", {})) | set(counters.get("WRITE_SIZE", {})))
        for k in kinds:
            fe = counters.get("FETCH_SIZE", {}).get(k, [])
            wr = counters.get("WRITE_SIZE", {}).get(k, [])
            fe_avg = sum(fe) / len(fe) if fe else 0.0
            wr_avg = sum(wr) / len(wr) if wr else 0.0
            b = None
            if "FETCH_SIZE" in factors and "WRITE_SIZE" in factors:
                b = fe_avg * 1024 * factors["FETCH_SIZE"] + wr_avg * 1024 * factors["WRITE_SIZE"]
                traffic[k] = {"bytes_per_launch": round(b), "fetch_kib": round(fe_avg, 1),
                              "write_kib": round(wr_avg, 1)}
            out.append(f"| {k} | {fe_avg:.1f} | {wr_avg:.1f} | "
                       f"{'-' if b is None else f'{b:.4g}'} |")
        for c, f in factors.items():
            out.append(f"\n{c} calibration: copy of {copy_bytes} bytes -> factor {f:.4f} "
                       "bytes per reported byte")
        out.append("")
        out.append("traffic-json: " + json.dumps(traffic))
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default=DEFAULT, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-vendor", action="store_true",
                    help="skip timing the same products with hipBLASLt (torch.mm)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="before the timed steps, run one device-to-device copy of BYTES "
                         "(reference kernel for HBM counter calibration)")
    ap.add_argument("--summarize", nargs="+", metavar="DIR",
                    help="print a markdown summary of rocprofv3 output directories and exit")
    ap.add_argument("--timed-steps", type=int, default=0, metavar="K",
                    help="with --summarize: also average each kernel over the last K steps")
    args = ap.parse_args()
    if args.summarize:
        print(summarize(args.summarize, args.copy_calibration, args.timed_steps))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path).", file=sys.stderr)
        sys.exit(2)

    import torch
    import orda_hip as H
    if not H.is_available():
        raise SystemExit("liborda_hip.so sees no gfx950 device")
    wl = WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    log(f"workload {args.workload}: generating inputs")
    s, w, y, t = make_inputs(torch, wl, dev)
    teacher = teacher_obj(H, t)
    opts = options(H, wl)
    ctx = H.Context(0)
    torch.cuda.synchronize()
    out = None
    for i in range(args.warmup):
        out = H.distillation_loss(s, w, y, teacher, opts, ctx=ctx)
        log(f"warmup {i + 1}/{args.warmup}: loss {out.loss:.5f}")
    outputs = {"grad_student_hidden": out.grad_student_hidden, "grad_weight": out.grad_weight}
    if out.grad_teacher_hidden is not None:
        outputs["grad_teacher_hidden"] = out.grad_teacher_hidden
    if out.grad_teacher_weight is not None:
        outputs["grad_teacher_weight"] = out.grad_teacher_weight
    plan = out.chunk_plan
    if args.copy_calibration:
        n = args.copy_calibration // 4
        src = torch.ones(n, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy of {n * 4} bytes done")
        del src, dst
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        out = H.distillation_loss(s, w, y, teacher, opts, ctx=ctx, outputs=outputs)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    log(f"timed {args.steps} steps in {elapsed * 1e3:.1f} ms, loss {out.loss:.5f}")
    # Per-kernel durations from the same number of steps run again with the
    # library's HIP events around every kernel (kept out of the timed steps:
    # they add ~0.3 % per step at this workload, ~10 % at BT=256).
    ctx.reset_timing()
    ctx.set_timing(True)
    for i in range(args.steps):
        out = H.distillation_loss(s, w, y, teacher, opts, ctx=ctx, outputs=outputs)
    torch.cuda.synchronize()
    ctx.set_timing(False)
    teacher_kind, bt, h, ht, v = wl[:5]
    dt = compute_dtype(wl)
    work = work_per_step(wl, plan)
    kernels = {}
    for kind, (bound, amount) in work.items():
        ms, n = ctx.kernel_time(kind)
        if n == 0 or amount == 0:
            continue
        per_step = amount
        if bound == "mfma":
            achieved = per_step * args.steps / (ms * 1e-3) / 1e12
            peak = PEAK_MFMA_TFLOPS[dt]
            unit = "TFLOP/s"
        else:
            achieved = per_step * args.steps / (ms * 1e-3) / 1e9
            peak = PEAK_HBM_GBS
            unit = "GB/s"
        kernels[kind] = {"bound": bound, "achieved": round(achieved, 2), "peak": peak,
                         "unit": unit, "frac": round(achieved / peak, 4),
                         "ms_per_step": round(ms / args.steps, 4),
                         "launches_per_step": n // args.steps,
                         "work_per_step": per_step}
    ms_other, _ = ctx.kernel_time("other")
    dom = max(kernels, key=lambda k: kernels[k]["ms_per_step"])
    d = kernels[dom]
    n_launch = max(d["launches_per_step"], 1)
    roofline = {"bound": d["bound"], "kernel": dom, "achieved": d["achieved"], "peak": d["peak"],
                "unit": d["unit"], "frac": d["frac"],
                "work_per_launch": d["work_per_step"] / n_launch,
                "avg_launch_ms": d["ms_per_step"] / n_launch,
                "traffic": read_traffic(args.workload, dom)}
    rows_per_s = bt * args.steps / elapsed
    line = {
        "metric": "fwd+bwd rows/sec at BT=8192 H=4096 V=131072; MFMA util %; row-pass HBM GB/s",
        "value": round(rows_per_s, 1), "unit": "rows/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(elapsed / args.steps * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": dt, "data": "synthetic",
        "config": {"workload": args.workload, "teacher": teacher_kind, "bt": bt, "h": h,
                   "v": v, "chunks": f"{plan.num_chunks}x{plan.chunk_size}",
                   "inputs": wl[5], "profile": profile_of(wl) or "balanced"},
        "roofline": roofline,
        "kernels": kernels,
        "mfma_util": {k: kernels[k]["frac"] for k in kernels if kernels[k]["bound"] == "mfma"},
        "row_pass_gbs": kernels.get("row_pass", {}).get("achieved"),
        "other_ms_per_step": round(ms_other / args.steps, 4),
    }
    del out, outputs
    ctx.close()
    torch.cuda.empty_cache()
    if not args.no_vendor:
        log("timing the same products with the vendor library")
        line["vendor_gemm"] = vendor_gemms(torch, wl, dev, s, w, t, args.steps)
    del s, w, y, t, teacher
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        log("timing the CPU oracle on a bounded sample")
        line["cpu_baseline"] = cpu_baseline(wl)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
