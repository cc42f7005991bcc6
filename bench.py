"""Benchmark of TinyBrainHIP's quantized matmul on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Default workload (BASELINE.json config 1 at M=1, the config the headline
metric "dequant-GEMV GB/s and % of HBM peak" is quoted on):
  INT4 weight-only GEMV, symmetric signed 4-bit, one fp32 scale per 32
  consecutive K elements (converter layout), x fp32 [1 x K], for the four
  shapes [N x K] = 2048x2048, 5632x2048, 2048x5632, 32000x2048.
  One step = one GEMV of each shape.  Weights rotate through a pool of
  distinct copies totalling >= 2 GiB so every launch streams from HBM rather
  than the 256 MiB Infinity Cache.  Inputs are resident in HBM before timing.

Exactly --warmup untimed steps run first, then exactly --steps timed steps,
each launched from HIP graphs of at most one pool sweep.
value = algorithmic bytes of all GEMVs in the timed steps / wall time (GB/s),
algorithmic bytes per GEMV = W + S + Z + 4*M*K + 4*M*N.
The roofline object reports the dominant kernel (32000x2048) timed with HIP
events on its own stream over back-to-back launches; they are that kernel's
last launches in the run, which ``--trace-summary`` averages from a rocprofv3
kernel trace.  cpu_baseline
times the restated reference CPU path (dequantize() single-threaded, then
sgemm on every host CPU this process may use, capped by the CPU share
OMP_NUM_THREADS grants) on a bounded sample of the same workload.  The
default line also carries "decode_1p1b_int8": tokens/s of the 1.1B-shaped
INT8 decode step (the headline metric's second half), same step counts,
and one key per remaining BASELINE row (TABLE below: INT8 configs[0],
INT4 configs[1] at M=4 and 8, configs[3] prefill INT8 M=2048 and INT4
M=512, configs[4] 7B projection set at M=1 and 8 and the 7B decode step),
each with its own roofline and a bounded CPU baseline sample (a fifth of
--cpu-budget); --no-table skips them.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s

WORKLOADS = {
    # name: (precision, group, shapes [(N, K)], M)
    "int4_g32_gemv_m1": ("int4", 32, [(2048, 2048), (5632, 2048), (2048, 5632), (32000, 2048)], 1),
    "int4_g32_gemv_m4": ("int4", 32, [(2048, 2048), (5632, 2048), (2048, 5632), (32000, 2048)], 4),
    "int4_g32_gemv_m8": ("int4", 32, [(2048, 2048), (5632, 2048), (2048, 5632), (32000, 2048)], 8),
    "int8_pc_gemv_m1": ("int8", 0, [(5632, 2048)], 1),
    # the same shapes in the runtime layout Tensor.quantize(.int4) writes
    # (groups of 32 along N of the [K, N] weight)
    "int4_g32_gemv_m1_runtime": ("int4kn", 32, [(2048, 2048), (5632, 2048), (2048, 5632), (32000, 2048)], 1),
}

# Prefill: x [M x K] bf16 N(0,1), one dequant-GEMM on
# bf16 MFMA per step.  name: (precision, group, (N, K), M)
PREFILL = {}
for _m in (64, 128, 512, 2048):
    PREFILL[f"prefill_int8_m{_m}"] = ("int8", 0, (5632, 2048), _m)
    PREFILL[f"prefill_int4_m{_m}"] = ("int4", 32, (2048, 5632), _m)
    # the INT4 shape in the runtime layout Tensor.quantize(.int4) writes
    PREFILL[f"prefill_int4kn_m{_m}"] = ("int4kn", 32, (2048, 5632), _m)
# The same products through the fp32 entry (tbh_matmul_device), the
# reference's own activation type: x [M x K] fp32 N(0,1).
PREFILL_F32 = {"prefill_f32_" + k[len("prefill_"):]: v for k, v in PREFILL.items()}
# Decode (BASELINE configs[2] and [4]): one token of a LLaMA-shaped model on
# the GPU decode step.  name: (precision, group, config kwargs, context)
CFG_7B = dict(num_layers=32, hidden=4096, num_heads=32, num_kv_heads=32, intermediate=11008, vocab=32000)
DECODE = {
    "decode_1p1b_int8": ("int8", 0, dict(num_layers=22, hidden=2048, num_heads=32, num_kv_heads=4,
                                         intermediate=5632, vocab=32000), 512),
    "decode_7b_int4": ("int4", 32, CFG_7B, 512),
}
# The per-token projection set of the 7B shape (batch
# M in {1, 8}): every layer's q, k, v, o, gate, up and down GEMV and the LM
# head, each with M rows of x, one step = one token for each of M sequences.
# name: (precision, group, config kwargs, M)
PROJ = {
    "proj_7b_int4_m1": ("int4", 32, CFG_7B, 1),
    "proj_7b_int4_m8": ("int4", 32, CFG_7B, 8),
}
# The same sets with every projection its own launch (7 per layer) instead
# of q|k|v and gate|up concatenated at repack (4 per layer).
PROJ_SEP = {name + "_sep": cfg for name, cfg in PROJ.items()}
# The other backend protocols (softmax, RMSNorm, SiLU/GELU, attention) at the
# shapes either side of the GEMV in a 1.1B-shaped model: one launch per step
# over a >= 2 GiB rotating pool of inputs.  name: (op, shape kwargs)
OPS = {
    "op_softmax_256x32000": ("softmax", dict(rows=256, cols=32000)),          # logits of 256 tokens
    "op_rmsnorm_2048x2048": ("rmsnorm", dict(rows=2048, hidden=2048)),        # 2048-token prefill
    "op_silu_2048x5632": ("silu", dict(n=2048 * 5632)),
    "op_gelu_2048x5632": ("gelu", dict(n=2048 * 5632)),
    "op_attention_decode_ctx4096": ("attention", dict(batch=1, seq=1, kv=4096, hd=64, nh=32, nkv=4)),
}
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
RIDGE_FLOP_PER_BYTE = MFMA_BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)

# The rest of the BASELINE table, measured after the headline workload and
# the 1.1B decode step in the default run, each as a key of the default line
# with its own roofline and a bounded CPU baseline sample.
TABLE = ["int8_pc_gemv_m1", "int4_g32_gemv_m4", "int4_g32_gemv_m8", "prefill_int8_m2048", "prefill_int4_m512",
         "proj_7b_int4_m1", "proj_7b_int4_m8", "decode_7b_int4"]

# What roofline.frac is computed from.
FRAC_BASIS_KERNEL = ("events: HIP events on the replay stream around graphs of back-to-back launches of "
                     "this kernel alone, so the per-launch time includes the gap between launches; the "
                     "rocprofv3 kernel trace under profiles/ (dispatch start to end) reads a few percent less")
FRAC_BASIS_CALL = ("events: HIP events around graphs of back-to-back calls, each call's launches (the "
                   "split-K sum included) and the gaps between them")
FRAC_BASIS_STEP = "events: HIP events around graph replays of whole steps, every launch and gap included"


def alg_bytes(prec: str, gs: int, N: int, K: int, M: int) -> int:
    if prec in ("int4", "int4kn"):
        w = (K * N + 1) // 2
        s = 4 * ((K * N + gs - 1) // gs)
    else:
        w = K * N
        s = 4 * N
    return w + s + 4 * M * K + 4 * M * N


def profiled_traffic(prec: str, N: int, K: int, M: int, kind: str = ""):
    """HBM bytes per launch of this kernel measured with rocprofv3 --pmc
    (FETCH_SIZE + WRITE_SIZE, calibrated against a streaming kernel of known
    size), as recorded in profiles/; None when no matching record exists.
    kind "prefill": the bf16 MFMA GEMM's record (bytes per matmul call, the
    split-K partial-sum launch included when the call makes one)."""
    path = os.path.join(ROOT, "profiles", f"traffic_{kind + '_' if kind else ''}{prec}_{N}x{K}_m{M}.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip())
    return None


def profiled_step_traffic(workload: str):
    """HBM bytes per step of a decode or projection-set workload measured with
    rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE summed over one step's launches,
    calibrated against a copy kernel of known size), as recorded in
    profiles/traffic_<workload>.txt; None when no record exists."""
    path = os.path.join(ROOT, "profiles", f"traffic_{workload}.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_step:"):
            return int(line.split(":", 1)[1].strip())
    return None


def pmc_copies(torch, dev):
    """The calibration kernel of a --pmc-pass run: 5 device-to-device copies
    of 64 MiB (64 MiB read and 64 MiB written per launch)."""
    src = torch.ones(16 << 20, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    return src.numel() * 4


def host_info() -> dict:
    """Host cores as this process sees them: nproc, the CPUs it may run on,
    the CPU share the environment grants (OMP_NUM_THREADS; 16 per GPU on the
    MI355X boxes) and the lscpu model name."""
    nproc = os.cpu_count() or 1
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = nproc
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    model = ""
    try:
        import subprocess

        for line in subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except Exception:
        pass
    return {"nproc": nproc, "affinity_cpus": aff, "omp_num_threads": share or None, "model": model}


def cpu_threads() -> int:
    """Threads for the CPU baseline's sgemm: every CPU this process may run
    on, capped by the CPU share the environment grants (OMP_NUM_THREADS)."""
    h = host_info()
    return max(1, min(h["affinity_cpus"], h["omp_num_threads"] or h["affinity_cpus"]))


def step_graphs(torch, stream, launch_step, n_steps: int, per_graph: int, first: int = 0):
    """HIP graphs that together launch steps first .. first + n_steps - 1
    (launch_step(i) enqueues step i on `stream`), at most per_graph steps per
    graph.  Returns the list of graphs in launch order."""
    graphs = []
    i = first
    while i < first + n_steps:
        n = min(per_graph, first + n_steps - i)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for j in range(i, i + n):
                launch_step(j)
        graphs.append(g)
        i += n
    return graphs


def make_weight(prec: str, gs: int, N: int, K: int, seed: int):
    """Synthetic W ~ N(0, 0.02) as PyTorch [N, K], quantized with the
    product's restatement of the reference quantizers."""
    import tinybrain_amd as T

    rng = np.random.default_rng(seed)
    w_nk = rng.normal(0.0, 0.02, size=(N, K)).astype(np.float32)
    if prec == "int4":
        return T.quantize_int4_flat(w_nk, gs, shape=(K, N), layout=T.Layout.NK_FLAT)
    if prec == "int4kn":     # runtime layout: [K, N] flattened, groups along N
        return T.quantize_int4_flat(np.ascontiguousarray(w_nk.T), gs, layout=T.Layout.KN_FLAT)
    return T.quantize(np.ascontiguousarray(w_nk.T), T.QuantizationMode.perChannel)


def host_entry(backend, pool, shapes, M: int, prec: str, gs: int, reps: int = 200) -> dict:
    """tbh_matmul as the Swift drop-in calls it: x and y in pageable host
    memory, the copy of x in, the copy of y out and the synchronisation
    inside every call (MetalBackend.matmulQuantized's commit-and-wait,
    MetalBackend.swift:894-974).  Weights rotate through the same >= 2 GiB
    pool, so every call streams its weight from HBM.  Median over `reps`
    calls per shape, after 10 untimed ones."""
    from tinybrain_amd import _abi

    lib = _abi.lib()
    rng = np.random.default_rng(3)
    per, total_us, total_b = {}, 0.0, 0
    for j, (N, K) in enumerate(shapes):
        x = rng.standard_normal((M, K), dtype=np.float32)
        y = np.empty((M, N), np.float32)
        ts = []
        for i in range(reps + 10):
            w = pool[i % len(pool)][j]
            t0 = time.perf_counter()
            st = lib.tbh_matmul(backend._dev, x.ctypes.data, M, K, w.handle, y.ctypes.data)
            t1 = time.perf_counter()
            if st != 0:
                raise RuntimeError(f"tbh_matmul: status {st}")
            if i >= 10:
                ts.append(t1 - t0)
        us = float(np.median(ts)) * 1e6
        b = alg_bytes(prec, gs, N, K, M)
        per[f"{N}x{K}"] = {"us": round(us, 2), "GB_s": round(b / us / 1e3, 1)}
        total_us += us
        total_b += b
    return {"entry": "tbh_matmul: host x and y (pageable), copies and synchronisation included",
            "per_shape": per, "us_per_step": round(total_us, 2), "GB_s": round(total_b / total_us / 1e3, 1),
            "calls_per_shape": reps}


def cpu_baseline(qts, shapes, M: int, budget_s: float = 15.0):
    """Reference CPU path (QuantizedTensor.swift:640-642) restated in the
    oracle: single-threaded dequantize() into a fresh fp32 [K, N] buffer, then
    sgemm on all host cores.  Times whole steps until ~budget_s."""
    import oracle as O

    threads = cpu_threads()
    oq = []
    for qt in qts:
        oq.append(O.QTensor(qt.shape, qt.data, qt.scales, qt.zeroPoints, int(qt.mode),
                            int(qt.precision), qt.groupSize))
    xs = {K: np.random.default_rng(1).normal(size=(M, K)).astype(np.float32) for _, K in shapes}
    steps = 0
    t_deq = t_gemm = 0.0
    byts = 0
    t0 = time.perf_counter()
    while True:
        for (N, K), q, qt in zip(shapes, oq, qts):
            _, td, tg = O.matmul_quantized_cpu(xs[K], q, threads=threads)
            t_deq += td
            t_gemm += tg
            byts += alg_bytes("int4" if qt.precision == 2 else "int8", qt.groupSize, N, K, M)
        steps += 1
        if time.perf_counter() - t0 > budget_s or steps >= 50:
            break
    wall = time.perf_counter() - t0
    return {
        "value": round(byts / wall / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "host": host_info(),
        "kind": "port",
        "sample": f"{steps} step(s) of the same workload (one GEMV per shape, M={M}); "
                  f"dequantize {t_deq:.2f}s single-threaded + sgemm {t_gemm:.2f}s on {threads} threads",
        "ms_per_step": round(1e3 * wall / steps, 3),
        "best_effort": cpu_best_effort(qts, oq, shapes, xs, M, threads, budget_s / 3),
    }


def cpu_best_effort(qts, oq, shapes, xs, M: int, threads: int, budget_s: float):
    """The host's upper bound beside the reference path: a fused dequant-GEMV
    (oracle orc_matmul_quantized_fused: each quantized element read once and
    dequantized in registers, all threads; not the reference's algorithm,
    same result bit for bit).  Whole steps until ~budget_s."""
    import oracle as O
    import tinybrain_amd as T

    steps, byts, t = 0, 0, 0.0
    t0 = time.perf_counter()
    while True:
        for (N, K), q, qt in zip(shapes, oq, qts):
            _, dt = O.matmul_quantized_fused(xs[K], q, threads=threads, nk=qt.layout == T.Layout.NK_FLAT)
            t += dt
            byts += alg_bytes("int4" if qt.precision == 2 else "int8", qt.groupSize, N, K, M)
        steps += 1
        if time.perf_counter() - t0 > budget_s or steps >= 200:
            break
    return {
        "value": round(byts / t / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "best-effort fused dequant-GEMV (not the reference path; an upper bound for the host)",
        "sample": f"{steps} step(s), M={M}",
        "ms_per_step": round(1e3 * t / steps, 3),
    }


def prefill_bytes(prec: str, gs: int, N: int, K: int, M: int, x_bytes: int = 2) -> int:
    """W + S + x_bytes*M*K (bf16 x, or 4 for fp32 x) + 4*M*N (fp32 y)."""
    return alg_bytes(prec, gs, N, K, 0) + x_bytes * M * K + 4 * M * N


def cpu_baseline_prefill(qt, N, K, M, budget_s: float = 15.0, bf16_x: bool = True):
    """Reference CPU path on the same product: dequantize() single-threaded,
    then sgemm of the fp32 activations (bf16-valued for a bf16 workload) on
    all host cores."""
    import oracle as O

    threads = cpu_threads()
    oq = O.QTensor(qt.shape, qt.data, qt.scales, qt.zeroPoints, int(qt.mode), int(qt.precision),
                   qt.groupSize)
    x = np.random.default_rng(1).normal(size=(M, K)).astype(np.float32)
    if bf16_x:
        x = (x.view(np.uint32) & 0xFFFF0000).view(np.float32)
    steps, t_deq, t_gemm = 0, 0.0, 0.0
    t0 = time.perf_counter()
    while True:
        _, td, tg = O.matmul_quantized_cpu(x, oq, threads=threads)
        t_deq += td
        t_gemm += tg
        steps += 1
        if time.perf_counter() - t0 > budget_s or steps >= 20:
            break
    wall = time.perf_counter() - t0
    return {
        "value": round(2.0 * M * N * K * steps / wall / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": threads,
        "host": host_info(),
        "kind": "port",
        "sample": f"{steps} GEMM(s) of the same shape; dequantize {t_deq:.2f}s single-threaded + "
                  f"sgemm {t_gemm:.2f}s on {threads} threads",
        "ms_per_step": round(1e3 * wall / steps, 3),
    }


def measure_prefill(args, backend, T, torch, workload, cpu_budget):
    """Prefill TFLOP/s of one PREFILL workload (graphs of back-to-back
    tbh_matmul_bf16_device calls over a >= 2 GiB weight pool) or PREFILL_F32
    workload (tbh_matmul_device with fp32 x).  Returns the result object (the
    bench line's fields)."""
    f32 = workload in PREFILL_F32
    prec, gs, (N, K), M = (PREFILL_F32 if f32 else PREFILL)[workload]
    matmul = backend.matmul_device if f32 else backend.matmul_bf16_device
    dev = torch.device("cuda", 0)
    t_setup = time.perf_counter()
    base = make_weight(prec, gs, N, K, seed=0x7B1A0030)
    n_sets = max(2, int(np.ceil(args.pool_gib * 2**30 / alg_bytes(prec, gs, N, K, 0))))
    pool = [T.DeviceWeight(backend, base) for _ in range(n_sets)]
    setup_s = time.perf_counter() - t_setup
    gen = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn((M, K), generator=gen, device=dev, dtype=torch.float32)
    if not f32:
        x = x.to(torch.bfloat16)
    y = torch.empty((M, N), device=dev, dtype=torch.float32)
    cap = torch.cuda.Stream(dev)
    cap.wait_stream(torch.cuda.current_stream(dev))
    if args.pmc_pass:
        src = torch.ones(16 << 20, dtype=torch.float32, device=dev)   # 64 MiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        for i in range(20):
            matmul(x, pool[i % n_sets], out=y, stream=cap)
        torch.cuda.synchronize()
        return {"pmc_pass": True, "copy_bytes": src.numel() * 4, "workload": workload,
                "alg_bytes_per_launch": prefill_bytes(prec, gs, N, K, M, 4 if f32 else 2)}
    for i in range(n_sets):
        matmul(x, pool[i], out=y, stream=cap)
    torch.cuda.synchronize()
    eager = y.clone()

    def step(i):
        matmul(x, pool[i % n_sets], out=y, stream=cap)

    check = step_graphs(torch, cap, step, n_sets, n_sets)[0]
    for _ in range(2):
        y.zero_()
        with torch.cuda.stream(cap):
            check.replay()
        torch.cuda.synchronize()
        if not torch.equal(y, eager):
            raise RuntimeError("graph replay differs from the eager launches")
    del check
    warm_graphs = step_graphs(torch, cap, step, args.warmup, n_sets)
    timed_graphs = step_graphs(torch, cap, step, args.steps, n_sets, first=args.warmup)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(cap):
        for g in warm_graphs:
            g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(cap)
        for g in timed_graphs:
            g.replay()
        e1.record(cap)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    steps_done = args.steps
    kern_us = e0.elapsed_time(e1) * 1e3 / steps_done
    flops = 2.0 * M * N * K
    byts = prefill_bytes(prec, gs, N, K, M, 4 if f32 else 2)
    value = flops * steps_done / wall / 1e12
    mfma_bound = flops / byts >= RIDGE_FLOP_PER_BYTE
    if mfma_bound:
        roof = {"bound": "mfma", "achieved": round(flops / kern_us / 1e6, 2),
                "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s"}
    else:
        roof = {"bound": "hbm", "achieved": round(byts / kern_us / 1e3, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    # past 64 rows (TBH_PREFILL_F16_MIN) the f16 forms: runtime-layout INT4
    # on the weight-side kernel, fp32 x as two f16 pieces
    f16 = M >= int(os.environ.get("TBH_PREFILL_F16_MIN") or 65) and (
        prec == "int4kn" or (f32 and os.environ.get("TBH_PREFILL_F32_PIECES") != "4"))
    kern = "gemm_ngw" if prec == "int4kn" and f16 else "gemm_bf16"
    x_form = ("fp32 x, two f16 pieces" if f16 else "fp32 x, three bf16 pieces") if f32 else "bf16 x"
    roof.update({"traffic": profiled_traffic(prec, N, K, M, "prefill_f32" if f32 else "prefill"),
                 "kernel": f"{kern} {N}x{K} M={M} ({pool[0].path}, {x_form})",
                 "kernel_us": round(kern_us, 3), "alg_bytes_per_launch": byts,
                 "flops_per_launch": int(flops), "frac_basis": FRAC_BASIS_CALL})
    out = {
        "metric": f"prefill dequant-GEMM TFLOP/s on {'f16' if f16 else 'bf16'} MFMA ({ {'int4kn': 'INT4 runtime layout'}.get(prec, prec.upper()) }, M={M}{', fp32 x' if f32 else ''})",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps_done,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * wall / steps_done, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if f16 else "bf16",
        "data": "synthetic",
        "config": {
            "workload": workload,
            "weights": {"int4": "INT4 symmetric, group 32 along K (converter layout)",
                        "int4kn": "INT4 symmetric, group 32 along N (runtime layout, Tensor.quantize(.int4))",
                        "int8": "INT8 symmetric per output channel"}[prec],
            "shape_NxK": f"{N}x{K}", "M": M,
            "x": ("fp32 N(0,1)" if f32 else "bf16 (rounded from fp32 N(0,1))") + ", W fp32 N(0,0.02) quantized",
            "pool_sets": n_sets,
        },
        "roofline": roof,
        "setup_s": round(setup_s, 1),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_prefill(base, N, K, M, cpu_budget, bf16_x=not f32)
    return out


def run_prefill(args, backend, T, torch):
    print(json.dumps(measure_prefill(args, backend, T, torch, args.workload, args.cpu_budget)), flush=True)
    backend.close()


def decode_shapes(c):
    """(K, N) of every projection of one layer, and of the LM head."""
    H, I, kv = c["hidden"], c["intermediate"], c["hidden"] // c["num_heads"] * c["num_kv_heads"]
    return [(H, H), (H, kv), (H, kv), (H, H), (H, I), (H, I), (I, H)], (H, c["vocab"])


def decode_bytes(prec, gs, c, ctx):
    """Algorithmic HBM bytes of one decode step: every GEMV's W + S + x + y,
    plus the K and V cache rows attention reads (fp32, ctx positions)."""
    layer, lm = decode_shapes(c)
    b = c["num_layers"] * sum(alg_bytes(prec, gs, N, K, 1) for K, N in layer)
    b += alg_bytes(prec, gs, lm[1], lm[0], 1)
    kv = c["hidden"] // c["num_heads"] * c["num_kv_heads"]
    return b + c["num_layers"] * 2 * ctx * kv * 4


def cpu_baseline_decode(prec, gs, c, qts, budget_s: float = 15.0, M: int = 1):
    """Reference CPU path for one step: every projection is dequantize()
    (single-threaded, fresh buffer) + sgemm of M rows on all host cores
    (QuantizedTensor.swift:640-642).  Timed on one layer's seven projections
    and the LM head; a step is num_layers layers + the LM head (attention,
    norms and activations, which the CPU path also runs, are left out) and
    yields M tokens."""
    import oracle as O

    threads = cpu_threads()
    layer, lm = decode_shapes(c)
    oq = [O.QTensor(q.shape, q.data, q.scales, q.zeroPoints, int(q.mode), int(q.precision), q.groupSize)
          for q in qts]
    t_layer = t_lm = 0.0
    reps = 0
    t0 = time.perf_counter()
    while True:
        for (K, N), q in zip(layer, oq[:7]):
            x = np.random.default_rng(K).normal(size=(M, K)).astype(np.float32)
            t1 = time.perf_counter()
            O.matmul_quantized_cpu(x, q, threads=threads)
            t_layer += time.perf_counter() - t1
        x = np.random.default_rng(7).normal(size=(M, lm[0])).astype(np.float32)
        t1 = time.perf_counter()
        O.matmul_quantized_cpu(x, oq[7], threads=threads)
        t_lm += time.perf_counter() - t1
        reps += 1
        if time.perf_counter() - t0 > budget_s or reps >= 5:
            break
    step_s = (c["num_layers"] * t_layer + t_lm) / reps
    # the host's upper bound: the same projections as a fused dequant-GEMV
    import tinybrain_amd as T
    be_layer = be_lm = 0.0
    be_reps = 0
    t0 = time.perf_counter()
    while True:
        for j, ((K, N), q) in enumerate(zip(layer + [lm], oq)):
            x = np.random.default_rng(K).normal(size=(M, K)).astype(np.float32)
            _, dt = O.matmul_quantized_fused(x, q, threads=threads, nk=qts[j].layout == T.Layout.NK_FLAT)
            if j < 7:
                be_layer += dt
            else:
                be_lm += dt
        be_reps += 1
        if time.perf_counter() - t0 > budget_s / 3 or be_reps >= 20:
            break
    be_step = (c["num_layers"] * be_layer + be_lm) / be_reps
    return {
        "value": round(M / step_s, 4),
        "unit": "tokens/s",
        "cores": threads,
        "host": host_info(),
        "kind": "port",
        "sample": f"{reps} pass(es) over one layer's 7 projections + the LM head at M={M}, scaled to "
                  f"{c['num_layers']} layers; projections only",
        "ms_per_step": round(1e3 * step_s, 1),
        "best_effort": {
            "value": round(M / be_step, 4), "unit": "tokens/s", "cores": threads,
            "kind": "best-effort fused dequant-GEMV (not the reference path; an upper bound for the host)",
            "sample": f"{be_reps} pass(es) over the same projections", "ms_per_step": round(1e3 * be_step, 1),
        },
    }


def measure_decode(args, backend, T, torch, workload, cpu_budget=None):
    """Decode tokens/s of one DECODE workload: a HIP graph of one step,
    replayed exactly args.warmup times untimed and args.steps times timed.
    Returns the result object (the bench line's fields)."""
    prec, gs, c, ctx = DECODE[workload]
    dev = torch.device("cuda", 0)
    need = ctx + args.warmup + args.steps + 8
    if args.max_seq and args.max_seq < need:
        raise SystemExit(f"--max-seq {args.max_seq} is below the {need} positions this run fills")
    cfg = T.DecoderConfig(max_seq=args.max_seq or need, **c)
    layer, lm = decode_shapes(c)
    t_setup = time.perf_counter()
    # One random init per projection shape; every layer gets its own device
    # copy, so a step streams all num_layers layers' weights from HBM.
    qts = [make_weight(prec, gs, N, K, seed=0x7B1A0040 + j) for j, (K, N) in enumerate(layer)]
    qts.append(make_weight(prec, gs, lm[1], lm[0], seed=0x7B1A0050))
    rng = np.random.default_rng(5)
    emb = rng.normal(0, 1, size=(c["vocab"], c["hidden"])).astype(np.float32)
    norm = lambda: (1.0 + 0.1 * rng.normal(size=c["hidden"])).astype(np.float32)
    dec = T.Decoder(backend, cfg, emb, norm(), qts[7])
    for l in range(c["num_layers"]):
        dec.set_layer(l, norm(), norm(), qts[:7])
    setup_s = time.perf_counter() - t_setup

    cap = torch.cuda.Stream(dev)
    logits = torch.empty(c["vocab"], dtype=torch.float32, device=dev)
    tok = 1
    if args.pmc_pass:
        # every attention block loads its range's cache rows before it reads
        # the position, so a step's traffic is that of context ctx whatever
        # the (zero-filled) cache holds: no fill steps
        dec.set_position(ctx)
        copy_bytes = pmc_copies(torch, dev)
        for _ in range(3):
            dec.step_device(tok, logits, cap)
        torch.cuda.synchronize()
        dec.close()
        return {"pmc_pass": True, "copy_bytes": copy_bytes, "workload": workload, "steps": 3,
                "launches_per_step": 6 * c["num_layers"] + 1,
                "alg_bytes_per_step": int(decode_bytes(prec, gs, c, ctx + 2))}
    for _ in range(ctx):                      # fill the KV cache: context `ctx`
        dec.step_device(tok, logits, cap)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        dec.step_device(tok, logits, cap)
    dec.set_position(ctx)                     # capture does not run the step
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(cap):
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(cap)
        for _ in range(args.steps):
            graph.replay()
        e1.record(cap)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    if dec.position != ctx + args.warmup + args.steps:
        raise RuntimeError("decode position did not advance once per replay")
    step_us = e0.elapsed_time(e1) * 1e3 / args.steps
    mean_ctx = ctx + args.warmup + (args.steps - 1) / 2.0 + 1
    byts = decode_bytes(prec, gs, c, mean_ctx)
    achieved = byts / step_us / 1e3
    out = {
        "metric": f"decode tokens/s, {c['num_layers']}-layer LLaMA shape ({prec.upper()}), 1 GPU",
        "tokens_per_s": round(args.steps / wall, 2),
        "value": round(args.steps / wall, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * wall / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": workload, **c, "context": ctx, "max_seq": cfg.max_seq,
            "weights": ("INT8 symmetric per output channel" if prec == "int8" else
                        "INT4 symmetric, group 32 along K (converter layout)") +
                       "; one random init per projection shape, a device copy per layer",
            "batch": 1, "launches_per_step": 6 * c["num_layers"] + 1,
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profiled_step_traffic(workload),
            "kernel": "decode step (graph of all launches)", "kernel_us": round(step_us, 2),
            "alg_bytes_per_launch": int(byts), "frac_basis": FRAC_BASIS_STEP,
        },
        "setup_s": round(setup_s, 1),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_decode(prec, gs, c, qts,
                                                  args.cpu_budget if cpu_budget is None else cpu_budget)
    dec.close()
    return out


def run_decode(args, backend, T, torch):
    out = measure_decode(args, backend, T, torch, args.workload)
    out.pop("tokens_per_s", None)
    print(json.dumps(out), flush=True)
    backend.close()


def measure_proj(args, backend, T, torch, workload, cpu_budget):
    """The 7B projection set at M rows: num_layers x (q, k, v, o, gate, up,
    down) + the LM head through tbh_matmul_device, captured in one HIP
    graph.  Every layer has its own device copy of its seven weights (one
    random init per shape), so a step streams the whole model from HBM.
    Returns the result object (the bench line's fields)."""
    separate = workload in PROJ_SEP
    prec, gs, c, M = PROJ_SEP[workload] if separate else PROJ[workload]
    dev = torch.device("cuda", 0)
    layer, lm = decode_shapes(c)
    t_setup = time.perf_counter()
    qts = [make_weight(prec, gs, N, K, seed=0x7B1A0040 + j) for j, (K, N) in enumerate(layer)]
    qts.append(make_weight(prec, gs, lm[1], lm[0], seed=0x7B1A0050))
    # launches of a layer: (K, N, parts); the parts of one launch read the
    # same x (q, k, v; gate, up) and are concatenated at repack unless the
    # workload runs every projection on its own
    groups = [[j] for j in range(7)] if separate else [[0, 1, 2], [3], [4, 5], [6]]
    launches = [(layer[g[0]][0], sum(layer[j][1] for j in g), g) for g in groups]

    def device_weight(g):
        return T.DeviceWeight(backend, qts[g[0]]) if len(g) == 1 else \
            T.DeviceWeight.concat(backend, [qts[j] for j in g])

    weights = [[device_weight(g) for _, _, g in launches] for _ in range(c["num_layers"])]
    head = T.DeviceWeight(backend, qts[7])
    setup_s = time.perf_counter() - t_setup
    shapes = [(K, N) for K, N, _ in launches] + [lm]
    gen = torch.Generator(device=dev).manual_seed(3)
    xs = {K: torch.randn((M, K), generator=gen, device=dev, dtype=torch.float32) for K, _ in shapes}
    ys = {N: torch.empty((M, N), device=dev, dtype=torch.float32) for _, N in shapes}
    cap = torch.cuda.Stream(dev)
    cap.wait_stream(torch.cuda.current_stream(dev))

    def step():
        for ws in weights:
            for (K, N, _), w in zip(launches, ws):
                backend.matmul_device(xs[K], w, out=ys[N], stream=cap)
        backend.matmul_device(xs[lm[0]], head, out=ys[lm[1]], stream=cap)

    if args.pmc_pass:
        step()                                # sizes the split-K workspace
        copy_bytes = pmc_copies(torch, dev)
        for _ in range(3):
            step()
        torch.cuda.synchronize()
        byts = c["num_layers"] * sum(alg_bytes(prec, gs, N, K, M) for K, N, _ in launches) + \
            alg_bytes(prec, gs, lm[1], lm[0], M)
        return {"pmc_pass": True, "copy_bytes": copy_bytes, "workload": workload, "steps": 3,
                "calls_per_step": len(launches) * c["num_layers"] + 1, "alg_bytes_per_step": int(byts)}

    step()                                    # eager: sizes the split-K workspace of `cap`
    torch.cuda.synchronize()
    eager = {N: y.clone() for N, y in ys.items()}
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        step()
    for _ in range(2):
        for y in ys.values():
            y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for N, y in ys.items():
            if not torch.equal(y, eager[N]):
                raise RuntimeError("graph replay differs from the eager launches")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(cap):
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(cap)
        for _ in range(args.steps):
            graph.replay()
        e1.record(cap)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    step_us = e0.elapsed_time(e1) * 1e3 / args.steps
    byts = c["num_layers"] * sum(alg_bytes(prec, gs, N, K, M) for K, N, _ in launches) + \
        alg_bytes(prec, gs, lm[1], lm[0], M)
    achieved = byts / step_us / 1e3
    out = {
        "metric": f"7B projection-set tokens/s at batch M={M} (INT4 g32), 1 GPU",
        "value": round(M * args.steps / wall, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * wall / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": workload, **c, "M": M,
            "weights": "INT4 symmetric, group 32 along K (converter layout); one random init per "
                       "projection shape, a device copy per layer",
            "step": "q, k, v, o, gate, up, down of every layer + LM head (no attention or norms)" +
                    ("; every projection its own launch" if separate else
                     "; q|k|v and gate|up concatenated at repack (one launch each, as the decode step)"),
            "launches_per_step": len(launches) * c["num_layers"] + 1,
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profiled_step_traffic(workload),
            "kernel": "projection step (graph of all launches)", "kernel_us": round(step_us, 2),
            "alg_bytes_per_launch": int(byts), "frac_basis": FRAC_BASIS_STEP,
        },
        "setup_s": round(setup_s, 1),
    }
    del graph, weights, head
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_decode(prec, gs, c, qts, cpu_budget, M=M)
    return out


def run_proj(args, backend, T, torch):
    print(json.dumps(measure_proj(args, backend, T, torch, args.workload, args.cpu_budget)), flush=True)
    backend.close()


def op_sizes(op, c):
    """(input floats, output floats, algorithmic bytes) of one launch: each
    input read once and each output written once."""
    if op == "softmax":
        n_in, n_out, extra = c["rows"] * c["cols"], c["rows"] * c["cols"], 0
    elif op == "rmsnorm":
        n_in, n_out, extra = c["rows"] * c["hidden"], c["rows"] * c["hidden"], c["hidden"]
    elif op in ("silu", "gelu"):
        n_in, n_out, extra = c["n"], c["n"], 0
    else:
        q = c["batch"] * c["seq"] * c["nh"] * c["hd"]
        kv = c["batch"] * c["kv"] * c["nkv"] * c["hd"]
        n_in, n_out, extra = q + 2 * kv, q, 0
    return n_in, n_out, 4 * (n_in + n_out + extra)


def cpu_baseline_op(op, c, budget_s):
    """The float64 oracle of the reference's CPU path (numpy, one thread) on
    the same shape, repeated until about budget_s seconds."""
    import oracle.ops_ref as R

    rng = np.random.default_rng(5)
    if op == "softmax":
        x = rng.normal(size=(c["rows"], c["cols"])).astype(np.float32)
        fn = lambda: R.softmax(x)
    elif op == "rmsnorm":
        x = rng.normal(size=(c["rows"], c["hidden"])).astype(np.float32)
        w = np.ones(c["hidden"], np.float32)
        fn = lambda: R.rmsnorm(x, w)
    elif op in ("silu", "gelu"):
        x = rng.normal(size=c["n"]).astype(np.float32)
        fn = lambda: getattr(R, op)(x)
    else:
        q = rng.normal(size=(c["batch"], c["seq"], c["nh"] * c["hd"])).astype(np.float32)
        k = rng.normal(size=(c["batch"], c["kv"], c["nkv"] * c["hd"])).astype(np.float32)
        fn = lambda: R.attention(q, k, k, None, c["hd"], c["nh"], c["nkv"])
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    bytes_per = op_sizes(op, c)[2]
    return {"value": round(bytes_per * n / el / 1e9, 3), "unit": "GB/s", "cores": 1, "host": host_info(),
            "kind": "port",
            "sample": f"{n} full launches of the same shape through oracle/ops_ref.py (numpy float64), "
                      f"{el:.1f} s"}


def run_op(args, backend, T, torch):
    op, c = OPS[args.workload]
    dev = torch.device("cuda", 0)
    n_in, n_out, byts = op_sizes(op, c)
    n_sets = max(2, int(np.ceil(args.pool_gib * 2**30 / (4 * (n_in + n_out)))))
    gen = torch.Generator(device=dev).manual_seed(4)
    ins = [torch.randn(n_in, generator=gen, device=dev, dtype=torch.float32) for _ in range(n_sets)]
    outs = [torch.empty(n_out, device=dev, dtype=torch.float32) for _ in range(n_sets)]
    g = torch.ones(c.get("hidden", 1), device=dev, dtype=torch.float32)
    cap = torch.cuda.Stream(dev)

    def launch(i):
        x, y = ins[i], outs[i]
        if op == "softmax":
            backend.softmax_device(x.view(c["rows"], c["cols"]), out=y.view(c["rows"], c["cols"]), stream=cap)
        elif op == "rmsnorm":
            backend.rmsnorm_device(x.view(c["rows"], c["hidden"]), g, 1e-5,
                                   out=y.view(c["rows"], c["hidden"]), stream=cap)
        elif op in ("silu", "gelu"):
            getattr(backend, op + "_device")(x, out=y, stream=cap)
        else:
            q_n = c["batch"] * c["seq"] * c["nh"] * c["hd"]
            kv_n = c["batch"] * c["kv"] * c["nkv"] * c["hd"]
            q = x[:q_n].view(c["batch"], c["seq"], c["nh"] * c["hd"])
            k = x[q_n:q_n + kv_n].view(c["batch"], c["kv"], c["nkv"] * c["hd"])
            v = x[q_n + kv_n:].view(c["batch"], c["kv"], c["nkv"] * c["hd"])
            backend.attention_device(q, k, v, None, c["hd"], c["nh"], c["nkv"],
                                     out=y.view(c["batch"], c["seq"], c["nh"] * c["hd"]), stream=cap)

    cap.wait_stream(torch.cuda.current_stream(dev))
    for i in range(n_sets):
        launch(i)
    torch.cuda.synchronize()
    eager = outs[0].clone()
    step = lambda i: launch(i % n_sets)
    check = step_graphs(torch, cap, step, n_sets, n_sets)[0]
    outs[0].zero_()
    with torch.cuda.stream(cap):
        check.replay()
    torch.cuda.synchronize()
    if not torch.equal(outs[0], eager):
        raise RuntimeError("graph replay differs from the eager launches")
    del check
    warm_graphs = step_graphs(torch, cap, step, args.warmup, n_sets)
    timed_graphs = step_graphs(torch, cap, step, args.steps, n_sets, first=args.warmup)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(cap):
        for g in warm_graphs:
            g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(cap)
        for g in timed_graphs:
            g.replay()
        e1.record(cap)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    steps_done = args.steps
    kern_us = e0.elapsed_time(e1) * 1e3 / steps_done
    achieved = byts / kern_us / 1e3
    out = {
        "metric": f"{op} GB/s (algorithmic bytes: inputs read once, outputs written once)",
        "value": round(byts * steps_done / wall / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps_done,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * wall / steps_done, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": args.workload, "op": op, **c, "pool_sets": n_sets},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": f"tbh_{op}", "kernel_us": round(kern_us, 3), "alg_bytes_per_launch": byts},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_op(op, c, args.cpu_budget)
    print(json.dumps(out), flush=True)
    backend.close()


def trace_summary(path: str, kernel_re: str, last: int) -> None:
    """Markdown summary of a rocprofv3 kernel-trace CSV: per kernel, calls and
    average / min / max duration over all dispatches; with --kernel and
    --last, also over the last `last` dispatches of the matching kernel (the
    launches a bench line's roofline kernel time is measured on: the dominant
    shape's timed graph replays are its final launches in the run)."""
    import csv
    import re

    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), r["Kernel_Name"],
                         int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    rows.sort()
    per = {}
    for _, name, d in rows:
        per.setdefault(name, []).append(d)
    print("| kernel | calls | avg us | min us | max us |")
    print("|---|---|---|---|---|")
    for name, ds in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        print(f"| `{name[:90]}` | {len(ds)} | {np.mean(ds) / 1e3:.3f} | {min(ds) / 1e3:.3f} | "
              f"{max(ds) / 1e3:.3f} |")
    if kernel_re and last > 0:
        match = [(t, n, d) for t, n, d in rows if re.search(kernel_re, n)]
        tail = [d for _, _, d in match[-last:]]
        print()
        print(f"Last {len(tail)} of {len(match)} dispatches matching `{kernel_re}`: "
              f"avg {np.mean(tail) / 1e3:.3f} us, median {np.median(tail) / 1e3:.3f} us, "
              f"min {min(tail) / 1e3:.3f} us, max {max(tail) / 1e3:.3f} us")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="int4_g32_gemv_m1",
                    choices=sorted(WORKLOADS) + sorted(PREFILL) + sorted(PREFILL_F32) + sorted(DECODE) + sorted(PROJ) +
                    sorted(PROJ_SEP) +
                    sorted(OPS))
    ap.add_argument("--pool-gib", type=float, default=2.2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--max-seq", type=int, default=0,
                    help="decode workloads: the decoder's cache length (default: the context plus the "
                         "steps replayed)")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--no-host-entry", action="store_true",
                    help="GEMV workloads: leave out the host-pointer (tbh_matmul) timing")
    ap.add_argument("--no-decode", action="store_true",
                    help="int4_g32_gemv_m1: leave out the 1.1B decode-step measurement")
    ap.add_argument("--no-table", action="store_true",
                    help="int4_g32_gemv_m1: leave out the other BASELINE rows (" + ", ".join(TABLE) + ")")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="summarise a rocprofv3 --kernel-trace CSV (no GPU work): per-kernel averages over "
                         "all dispatches and over the last --last dispatches of kernels matching --kernel")
    ap.add_argument("--kernel", default="", help="--trace-summary: kernel-name regex")
    ap.add_argument("--last", type=int, default=0, help="--trace-summary: trailing dispatches to average")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="for rocprofv3 --pmc: 5 plain copies of 64 MiB (calibration kernel of "
                         "known size) then 20 launches of the dominant GEMV (of the GEMM for a "
                         "prefill workload; 3 eager steps for a decode or projection-set workload); "
                         "no timing")
    args = ap.parse_args()

    if args.trace_summary:
        return trace_summary(args.trace_summary, args.kernel, args.last)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the GEMV would shard along N "
                                   "(each GPU a share of the output rows, outputs all-gathered), but no "
                                   "multi-GPU path is built", "n_gpus": args.gpus}))
        sys.exit(2)

    import torch
    import tinybrain_amd as T

    torch.cuda.set_device(0)
    backend = T.HIPBackend(0)
    if args.workload in PREFILL or args.workload in PREFILL_F32:
        return run_prefill(args, backend, T, torch)
    if args.workload in DECODE:
        return run_decode(args, backend, T, torch)
    if args.workload in PROJ or args.workload in PROJ_SEP:
        return run_proj(args, backend, T, torch)
    if args.workload in OPS:
        return run_op(args, backend, T, torch)
    out = measure_gemv(args, backend, T, torch, args.workload, args.cpu_budget, with_host_entry=not args.no_host_entry)
    if args.workload == "int4_g32_gemv_m1" and not args.pmc_pass:
        if not args.no_decode:
            # the second half of the headline metric: decode tokens/s at the
            # 1.1B shape, same --steps / --warmup
            _release(torch)
            out["decode_1p1b_int8"] = measure_decode(args, backend, T, torch, "decode_1p1b_int8")
        if not args.no_table:
            # the rest of the BASELINE table, each row with its roofline and a
            # bounded sample of the reference CPU path
            budget = args.cpu_budget / 5
            for name in TABLE:
                _release(torch)
                if name in WORKLOADS:
                    r = measure_gemv(args, backend, T, torch, name, budget, with_host_entry=False)
                elif name in PREFILL:
                    r = measure_prefill(args, backend, T, torch, name, budget)
                elif name in DECODE:
                    r = measure_decode(args, backend, T, torch, name, budget)
                    r.pop("tokens_per_s")
                else:
                    r = measure_proj(args, backend, T, torch, name, budget)
                out[name] = r
    print(json.dumps(out), flush=True)
    backend.close()


def _release(torch):
    """Let the previous measurement's pool go before the next one allocates."""
    import gc

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def measure_gemv(args, backend, T, torch, workload, cpu_budget, with_host_entry=True):
    """GB/s of one WORKLOADS entry: one GEMV of each shape per step, graphs of
    back-to-back tbh_matmul_device calls over a >= 2 GiB weight pool.
    Returns the result object (the bench line's fields)."""
    prec, gs, shapes, M = WORKLOADS[workload]

    # ---- weights: one quantized base per shape, copied into a >= 2 GiB pool
    t_setup = time.perf_counter()
    bases = [make_weight(prec, gs, N, K, seed=0x7B1A0010 + i) for i, (N, K) in enumerate(shapes)]
    set_bytes = sum(alg_bytes(prec, gs, N, K, 0) for N, K in shapes)
    n_sets = max(2, int(np.ceil(args.pool_gib * 2**30 / set_bytes)))
    pool = [[T.DeviceWeight(backend, b) for b in bases] for _ in range(n_sets)]
    pool_bytes = sum(w.device_bytes for s in pool for w in s)
    setup_s = time.perf_counter() - t_setup

    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(2)
    xs = {K: torch.randn((M, K), generator=gen, device=dev, dtype=torch.float32) for _, K in shapes}
    ys = [torch.empty((M, N), device=dev, dtype=torch.float32) for N, _ in shapes]
    stream = torch.cuda.current_stream(dev)

    if args.pmc_pass:
        src = torch.ones(16 << 20, dtype=torch.float32, device=dev)   # 64 MiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        jd = int(np.argmax([alg_bytes(prec, gs, N, K, M) for N, K in shapes]))
        Nd, Kd = shapes[jd]
        for i in range(20):
            backend.matmul_device(xs[Kd], pool[i % n_sets][jd], out=ys[jd], stream=stream)
        torch.cuda.synchronize()
        return {"pmc_pass": True, "copy_bytes": src.numel() * 4, "kernel": f"{Nd}x{Kd}",
                "alg_bytes_per_launch": alg_bytes(prec, gs, Nd, Kd, M)}

    # Launches are captured into HIP graphs, so the timed region measures the
    # GPU, not Python/ctypes launch overhead.  Step i runs one GEMV of each
    # shape on pool set i mod n_sets.  Replays are checked against an eager
    # run on the capture stream (which also sizes that stream's split-K
    # workspace, so the captured launches split K exactly as the eager ones).
    cap = torch.cuda.Stream(dev)
    cap.wait_stream(stream)

    def step(i):
        ws = pool[i % n_sets]
        for j, (N, K) in enumerate(shapes):
            backend.matmul_device(xs[K], ws[j], out=ys[j], stream=cap)

    for i in range(n_sets):
        step(i)
    torch.cuda.synchronize()
    eager = [y.clone() for y in ys]
    # exactly `warmup` untimed steps, then exactly `steps` timed steps
    # (continuing the rotation), in graphs of at most one pool sweep each
    warm_graphs = step_graphs(torch, cap, step, args.warmup, n_sets)
    timed_graphs = step_graphs(torch, cap, step, args.steps, n_sets, first=args.warmup)
    check = step_graphs(torch, cap, step, n_sets, n_sets)[0]
    for r in range(2):
        for y in ys:
            y.zero_()
        with torch.cuda.stream(cap):
            check.replay()
        torch.cuda.synchronize()
        for y, e in zip(ys, eager):
            if not torch.equal(y, e):
                raise RuntimeError("graph replay differs from the eager launches")
    del check

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(cap):
        for g in warm_graphs:
            g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(cap)
        for g in timed_graphs:
            g.replay()
        e1.record(cap)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    steps_done = args.steps
    step_bytes = sum(alg_bytes(prec, gs, N, K, M) for N, K in shapes)
    value = step_bytes * steps_done / wall / 1e9
    gpu_step_us = e0.elapsed_time(e1) * 1e3 / steps_done
    del warm_graphs, timed_graphs

    # ---- per-shape kernel time: a graph of n_sets back-to-back launches of
    # one shape, bracketed by HIP events on the replay stream
    per_shape = {}
    shape_us, shape_n = {}, {}
    jd = int(np.argmax([alg_bytes(prec, gs, N, K, M) for N, K in shapes]))
    for j, (N, K) in enumerate(shapes):
        g1 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g1, stream=cap):
            for i in range(n_sets):
                backend.matmul_device(xs[K], pool[i][j], out=ys[j], stream=cap)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        nrep = max(3, 400 // n_sets)
        # graph.replay() launches on torch's current stream: make that the
        # stream the events are recorded on
        with torch.cuda.stream(cap):
            g1.replay()
            torch.cuda.synchronize()
            e0.record(cap)
            for _ in range(nrep):
                g1.replay()
            e1.record(cap)
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (nrep * n_sets)
        b = alg_bytes(prec, gs, N, K, M)
        shape_us[j] = us
        shape_n[j] = nrep * n_sets
        per_shape[f"{N}x{K}"] = {"us": round(us, 3), "GB_s": round(b / us / 1e3, 1),
                                 "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                                 "path": pool[0][j].path}
    Nd, Kd = shapes[jd]
    kern_us = shape_us[jd]
    kbytes = alg_bytes(prec, gs, Nd, Kd, M)
    achieved = kbytes / (kern_us * 1e-6) / 1e9
    traffic = profiled_traffic(prec, Nd, Kd, M)

    out = {
        "metric": (f"dequant-GEMV GB/s and % of HBM peak (INT4 g32, M={M}, 4 BASELINE shapes)"
                   if prec == "int4" else
                   f"dequant-GEMV GB/s and % of HBM peak (INT4 g32 runtime layout, M={M}, 4 BASELINE shapes)"
                   if prec == "int4kn" else f"dequant-GEMV GB/s and % of HBM peak (INT8 per-channel, M={M})"),
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps_done,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * wall / steps_done, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": workload,
            "weights": {"int4": "INT4 symmetric, group 32 along K (converter layout)",
                        "int4kn": "INT4 symmetric, group 32 along N (runtime layout, Tensor.quantize(.int4))",
                        "int8": "INT8 symmetric per output channel"}[prec],
            "shapes_NxK": [f"{N}x{K}" for N, K in shapes],
            "gpu_us_per_step": round(gpu_step_us, 3),
            "M": M,
            "x": "fp32 N(0,1), W fp32 N(0,0.02) quantized",
            "pool_bytes": pool_bytes,
            "pool_sets": n_sets,
            "frac_hbm_wall": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": f"{Nd}x{Kd} ({pool[0][jd].path})",
            "kernel_us": round(kern_us, 3),
            "alg_bytes_per_launch": kbytes,
            "timed_dispatches": shape_n[jd],
            "frac_basis": FRAC_BASIS_KERNEL,
        },
        "per_shape": per_shape,
        "setup_s": round(setup_s, 1),
    }
    if with_host_entry:
        out["host_entry"] = host_entry(backend, pool, shapes, M, prec, gs)
    del pool
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(bases, shapes, M, cpu_budget)
    return out


if __name__ == "__main__":
    main()
