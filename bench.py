"""Benchmark of the FP8 compute path on one MI355X (the workloads of BASELINE.json).

Headline ("step" = one e5ma_gemm call): the 8192^3 E5M2 x E4M3 -> BF16 GEMM (TN, per-tensor
scale_inv 1/64, inputs N(0,1)*8 with 0.01 % set to the largest finite value), reported in TFLOP/s and as
a fraction of the FP8 dense matrix-core peak.  Secondary lines (same JSON object, "secondary"): the
same GEMM with E5M2 x E5M2 and E5M2 x BF16 operands, the three TE backward GEMMs of config 4 (dgrad,
wgrad into an FP32 main_grad, dgrad with E5M2 output), GEMV 8192 x 8192 at batch 1 and 8 (weights rotated
through 6 distinct buffers so the 256 MB Infinity Cache cannot serve them), the fused AdamW step over
256M parameters (BF16 and FP32 state, E5M2 copy) and the 8192^2 FP32 -> E5M2 cast.

Every rate is algorithmic work / kernel time, the kernel time taken with HIP events on the stream the
kernels run on (torch's current stream) around K back-to-back calls.  "copy" times torch's device copy
of 1 GiB: the streaming rate this GPU reaches in practice, and the known-size kernel the HBM counters
are calibrated on.  roofline.traffic (HBM bytes per launch) comes from profiles/hbm_traffic.json, the
rocprofv3 FETCH_SIZE / WRITE_SIZE counters of each workload's kernel scaled by the copy's
calibration; null where no counter run covers the workload.  cpu_baseline: the oracle's FP32
FFMA-chain GEMM (oracle/e5ma_oracle.c, the reference's host emulation order) timed on this host on a
slab of output rows and scaled to the full problem.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only gemm,te,gemv,adam,cast,copy] [--no-cpu]
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP8_PEAK_TFLOPS = 5000.0    # MI355X dense FP8 matrix cores
BF16_PEAK_TFLOPS = 2500.0   # dense BF16
HBM_PEAK_GBS = 8000.0       # HBM3E
E4M3, BF16, FP16, FP32, E5M2 = 0, 1, 2, 3, 4
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.json")
SETTLE_S = 0.25  # headline calls run this long before its W warm-up calls (clock settling)
SETTLE_2ND_S = 0.1  # the same for each secondary GEMM line


def traffic_table():
    """Workload id -> HBM bytes per launch, from the committed counter summary (empty if absent)."""
    try:
        with open(TRAFFIC_FILE) as fh:
            return {k: v["hbm_bytes_per_launch"] for k, v in json.load(fh)["workloads"].items()}
    except (OSError, KeyError, ValueError):
        return {}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=30)  # the clock under FP8 matrix load settles in ~20 ms
    p.add_argument("--only", default="gemm,te,gemv,adam,cast,copy")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                   help="print per-(kernel, grid) duration statistics of a rocprofv3 kernel trace and exit")
    p.add_argument("--counters", metavar="COUNTER_COLLECTION_CSV",
                   help="with --trace-summary: per-kernel means of the counters of a rocprofv3 --pmc run")
    p.add_argument("--traffic-json", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                   help="print the HBM traffic table from a FETCH_SIZE and a WRITE_SIZE counter run and exit")
    return p.parse_args()


def short_kernel_name(name):
    """A kernel's name without 'void', namespaces and the argument list."""
    if name.startswith("void "):
        name = name[5:]
    for ns in ("e5ma::(anonymous namespace)::", "(anonymous namespace)::"):
        name = name.replace(ns, "")
    depth, cut = 0, len(name)
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            cut = i
            break
    return name[:cut]


def trace_summary(trace_csv, counters_csv=None):
    """Per (kernel, grid): dispatches, median / mean / min / max duration (us), registers, LDS.  With a
    counter CSV (rocprofv3 --pmc with --kernel-trace): per-kernel means of each counter over its
    dispatches, and for GRBM_GUI_ACTIVE the clock (cycles / 8 XCDs / duration) and, with
    SQ_VALU_MFMA_BUSY_CYCLES, the matrix cores' busy fraction (over 1024 SIMDs)."""
    import csv
    import statistics
    csv.field_size_limit(10**9)
    rows = list(csv.DictReader(open(trace_csv)))
    groups, dur_of = {}, {}
    for r in rows:
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        dur_of[r["Dispatch_Id"]] = d
        grid = int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"]))
        key = (short_kernel_name(r["Kernel_Name"]), grid)
        groups.setdefault(key, {"d": [], "r": r})["d"].append(d)
    print(f"source: {trace_csv} ({len(rows)} dispatches); durations in microseconds")
    print(f"{'kernel':<58} {'grid':>7} {'calls':>6} {'median':>9} {'mean':>9} {'min':>9} {'max':>9} "
          f"{'vgpr':>5} {'agpr':>5} {'lds':>7}")
    for (name, grid), g in sorted(groups.items(), key=lambda kv: -sum(kv[1]["d"])):
        d, r = g["d"], g["r"]
        print(f"{name[:58]:<58} {grid:>7} {len(d):>6} {statistics.median(d):>9.2f} {sum(d) / len(d):>9.2f} "
              f"{min(d):>9.2f} {max(d):>9.2f} {r.get('VGPR_Count', ''):>5} {r.get('Accum_VGPR_Count', ''):>5} "
              f"{r.get('LDS_Block_Size', ''):>7}")
    if counters_csv:
        kern = counter_means(counters_csv)
        print(f"\ncounters: {counters_csv} (means over the dispatches of each kernel and grid; the clock is "
              f"GRBM_GUI_ACTIVE / 8 XCDs / kernel duration, meaningful for kernels of many microseconds only)")
        for (name, grid), lst in sorted(kern.items()):
            names = sorted({c for _, cs in lst for c in cs})
            means = {c: sum(cs.get(c, 0.0) for _, cs in lst) / len(lst) for c in names}
            line = f"{name[:58]:<58} {grid:>7} n={len(lst):<4}" + "".join(f" {c}={means[c]:.4g}" for c in names)
            if "GRBM_GUI_ACTIVE" in means:
                clocks, busy = [], []
                for disp, cs in lst:
                    if disp in dur_of and dur_of[disp] > 0:
                        cyc = cs.get("GRBM_GUI_ACTIVE", 0.0) / 8
                        clocks.append(cyc / (dur_of[disp] * 1e3))
                        if "SQ_VALU_MFMA_BUSY_CYCLES" in cs and cyc > 0:
                            busy.append(cs["SQ_VALU_MFMA_BUSY_CYCLES"] / (1024 * cyc))
                if clocks:
                    line += (f"  clock GHz min/median/max {min(clocks):.3f}/{statistics.median(clocks):.3f}/"
                             f"{max(clocks):.3f}")
                if busy:
                    line += (f"  mfma busy % min/median/max {100 * min(busy):.1f}/{100 * statistics.median(busy):.1f}/"
                             f"{100 * max(busy):.1f}")
            print(line)


def counter_means(counters_csv):
    """(kernel, grid) -> [(dispatch id, {counter: value summed over its instances})] of a rocprofv3 --pmc
    counter collection CSV."""
    import csv
    csv.field_size_limit(10**9)
    per = {}
    for r in csv.DictReader(open(counters_csv)):
        grid = int(r["Grid_Size"]) // max(1, int(r["Workgroup_Size"]))
        key = (short_kernel_name(r["Kernel_Name"]), grid, r["Dispatch_Id"])
        per.setdefault(key, {}).setdefault(r["Counter_Name"], 0.0)
        per[key][r["Counter_Name"]] += float(r["Counter_Value"])
    kern = {}
    for (name, grid, disp), cs in per.items():
        kern.setdefault((name, grid), []).append((disp, cs))
    return kern


# The kernels (short name, grid) one launch of each workload runs, at bench.py's shapes (the GEMM kernels are
# persistent: at most one block per CU, 256 on the MI355X)
WORKLOAD_KERNELS = {
    "gemm_8192_e5m2xe4m3": [("f8k::gemm_f8_kernel<4, 0, true, true, 0>", 256)],
    "gemm_8192_e5m2xe5m2": [("f8k::gemm_f8_kernel<4, 4, true, true, 0>", 256)],
    "gemm_8192_e5m2xbf16": [("hk::gemm_h_kernel<4, 1, true, true, 0>", 256)],
    "gemm_8192_nn": [("f8k::gemm_f8_kernel<4, 0, false, true, 0>", 256)],
    "gemm_8192_nt": [("f8k::gemm_f8_kernel<4, 0, false, false, 0>", 256)],
    "gemm_8192_tt": [("f8k::gemm_f8_kernel<4, 0, true, false, 0>", 256)],
    "te_dgrad": [("f8k::gemm_f8_kernel<0, 4, false, true, 0>", 256)],
    "te_wgrad": [("f8k::gemm_f8_kernel<4, 0, false, false, 1>", 256)],
    "te_wgrad_tn": [("f8k::gemm_f8_kernel<0, 4, true, true, 1>", 256)],
    "te_dgrad_e5m2": [("f8k::gemm_f8_kernel<0, 4, false, true, 1>", 256)],
    "gemv_8192_n1": [("gemv_xlds_kernel<4, 1, 1, 2, 4>", 512)],
    "gemv_8192_n8": [("gemv_mfma_kernel<4, 1, 8, 2>", 512)],
    "gemv_65536x8192_n1": [("gemv_xlds_kernel<4, 1, 1, 2, 4>", 4096)],
    "adamw_256m_bf16": [("adam_kernel<1, 1, 1, 4, true>", 131072)],
    "adamw_256m_fp32": [("adam_kernel<3, 3, 3, 4, true>", 32768)],
    "cast_8192sq_fp32_e5m2": [("cast_kernel<3, 4, true, true>", 16384)],
    "cast_8192sq_fp32_e4m3": [("cast_kernel<3, 0, true, true>", 16384)],
    "quantize_8192sq_fp32_e5m2_tensor": [("q_clear_kernel", 1), ("q_amax_kernel<3, true>", 512),
                                         ("q_cast_kernel<3, 4, true>", 16384), ("q_finish_kernel", 1)],
    "quantize_8192sq_fp32_e4m3_rows": [("q_rows_blk_kernel<3, 0, 2>", 8192)],
    "copy_1gib": [("__amd_rocclr_copyBuffer", 256)],
}


def traffic_json(fetch_csv, write_csv):
    """The HBM traffic table bench.py reads (profiles/hbm_traffic.json), from a FETCH_SIZE and a
    WRITE_SIZE counter run of bench.py: per workload the KiB per launch of its kernels, scaled by what
    the counters read for the 1 GiB device copy (1 GiB read, 1 GiB written)."""
    fe = {k: sum(cs.get("FETCH_SIZE", 0.0) for _, cs in v) / len(v) for k, v in counter_means(fetch_csv).items()}
    wr = {k: sum(cs.get("WRITE_SIZE", 0.0) for _, cs in v) / len(v) for k, v in counter_means(write_csv).items()}
    copy = WORKLOAD_KERNELS["copy_1gib"][0]
    ff, wf = 2**30 / (fe[copy] * 1024), 2**30 / (wr[copy] * 1024)
    out = {"fetch_factor": round(ff, 4), "write_factor": round(wf, 4),
           "source": {"fetch": os.path.basename(fetch_csv), "write": os.path.basename(write_csv)}, "workloads": {}}
    for wid, ks in WORKLOAD_KERNELS.items():
        if not all(k in fe and k in wr for k in ks):
            continue
        fk, wk = sum(fe[k] for k in ks), sum(wr[k] for k in ks)
        out["workloads"][wid] = {"kernels": [f"{n} x{g}" for n, g in ks], "fetch_kib": round(fk, 1),
                                 "write_kib": round(wk, 1), "hbm_bytes_per_launch": round(fk * 1024 * ff + wk * 1024 * wf)}
    print(json.dumps(out, indent=1))


def progress(msg):
    """One line on stderr per finished part, so a long run shows where it is (stdout keeps the JSON)."""
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def host_cpu():
    """(CPU model, logical CPUs visible, threads used): at most 16, a one-GPU box's CPU share."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    n = os.cpu_count() or 1
    return model, n, max(1, min(16, n))


def cpu_baselines(only):
    """CPU figures beside the GPU lines: the reference's CPU semantics (the oracle's C restatement, or
    the reference's own MAC model where noted) on this host, at 1 thread and at `threads` threads.
    Returns (the headline's cpu_baseline object, a list of per-workload objects).  Each is a bounded
    sample of the workload (stated), its rate scaled to the workload's unit."""
    import numpy as np
    import oracle
    model, ncpu, threads = host_cpu()
    host = {"cpu_model": model, "logical_cpus": ncpu}
    rng = np.random.default_rng(1)

    def rate(fn, work, min_s=1.0):
        """(work units per second) of fn(), repeated until min_s elapsed"""
        t0, reps = time.perf_counter(), 0
        while True:
            fn()
            reps += 1
            dt = time.perf_counter() - t0
            if dt >= min_s:
                return work * reps / dt

    def line(wid, workload, unit, scale, sample, kind, f1, fn_all, work):
        v1, vn = rate(f1, work), rate(fn_all, work)
        progress(f"cpu baseline {wid} done")
        return {"id": wid, "workload": workload, "unit": unit, "value": round(vn * scale, 6),
                "value_1_thread": round(v1 * scale, 6), "cores": threads, "kind": kind, "sample": sample, **host}

    out = []
    headline = None
    if "gemm" in only:
        # the 8192^3 E5M2 x E4M3 GEMM as the reference's host emulation (ascending-k FP32 fmaf chain,
        # tests/test_util.h:119-144): a slab of output rows, rate scaled to the full problem
        Md = Nd = Kd = 8192
        A = np.tile(oracle.encode(E5M2, (rng.standard_normal(Kd * 64) * 8).astype(np.float32)), Md // 64)
        B = np.tile(oracle.encode(E4M3, (rng.standard_normal(Kd * 64) * 8).astype(np.float32)), Nd // 64)
        gm = oracle.Gemm(1, 0, Md, Nd, Kd, 1.0, E5M2, A, Kd, E4M3, B, Kd, sa=[1 / 64], sb=[1 / 64], ddt=BF16)
        r1, rn = 1, 16
        l = line("gemm_8192_e5m2xe4m3", "gemm 8192^3 E5M2 x E4M3 -> BF16 (fmaf chain)", "TFLOP/s", 1e-12,
                 f"{r1} (1 thread) / {rn} ({threads} threads) of 8192 output rows per run", "port",
                 lambda: gm.chain(rows=(0, r1), threads=1), lambda: gm.chain(rows=(0, rn), threads=threads),
                 2.0 * Nd * Kd)
        # rate() above used the same work per call for both; correct the all-thread figure to rn rows
        l["value"] = round(l["value"] * rn / r1, 6)
        headline = {k: l[k] for k in ("value", "unit", "cores", "kind", "sample")}
        headline.update(value_1_thread=l["value_1_thread"], **host)
        out.append(l)
        # 512^3 E5M2 x E5M2 -> BF16, N(0,1)*4, as the reference's MAC chain (BF16
        # accumulator, one rounding per MAC) -- with the reference's own lane model when it was built --
        # and as the fmaf chain
        M = N = K = 512
        a = oracle.encode(E5M2, (rng.standard_normal(M * K) * 4).astype(np.float32))
        b = oracle.encode(E5M2, (rng.standard_normal(K * N) * 4).astype(np.float32))
        ref = oracle.ref_library()
        fn = ref.ref_lane if ref is not None else None
        kind = "reference" if fn is not None else "port"
        rows1, rowsn = 2, 2 * threads
        l = line("gemm_512_lane_chain", "config 1: 512^3 E5M2 x E5M2 -> BF16, BF16-accumulating lane chain "
                 "(tests/e5m2effma_ref.h:114-129)", "GFLOP/s", 1e-9,
                 f"{rows1} (1 thread) / {rowsn} ({threads} threads) of 512 output rows per run"
                 + ("; the reference's ref_lane compiled from its sources" if fn else "; the oracle's lane"), kind,
                 lambda: oracle.lane_gemm(a, b, M, N, K, 1, 1, fn=fn, rows=(0, rows1)),
                 lambda: oracle.lane_gemm(a, b, M, N, K, 1, 1, fn=fn, rows=(0, rowsn), threads=threads),
                 2.0 * rows1 * N * K)
        l["value"] = round(l["value"] * rowsn / rows1, 6)
        out.append(l)
        # column-major mapping of the row-major product (e5ma_gemm(N, N, 512, 512, 512, A := b, B := a))
        g1 = oracle.Gemm(0, 0, M, N, K, 1.0, E5M2, b, M, E5M2, a, K, ddt=BF16)
        out.append(line("gemm_512_fmaf_chain", "config 1: 512^3 E5M2 x E5M2 -> BF16, fmaf chain", "GFLOP/s", 1e-9,
                        "the whole 512^3 product", "port", lambda: g1.chain(threads=1),
                        lambda: g1.chain(threads=threads), 2.0 * M * N * K))
    if "gemv" in only:
        Md = Kd = 8192
        W = oracle.encode(E5M2, (rng.standard_normal(Md * Kd) * 0.02 * 64).astype(np.float32))
        sa = np.full(Md, 1 / 64, np.float32)
        for n in (1, 8):
            x = oracle.encode(BF16, rng.standard_normal(Kd * n).astype(np.float32))
            g = oracle.Gemm(1, 0, Md, n, Kd, 1.0, E5M2, W, Kd, BF16, x, Kd, sa=sa, sa_vec=True, ddt=BF16)
            nbytes = Md * Kd + Md * 4 + Kd * n * 2 + Md * n * 2
            out.append(line(f"gemv_8192_n{n}", f"gemv 8192^2 E5M2 x BF16 n={n} (fmaf chain)", "GB/s", 1e-9,
                            "the whole 8192 x 8192 GEMV", "port", lambda g=g: g.chain(threads=1),
                            lambda g=g: g.chain(threads=threads), nbytes))
    if "cast" in only:
        n = 8192 * 8192
        x = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.02))
        qs = 57344.0 / float(np.abs(x).max())
        parts = np.linspace(0, n, threads + 1).astype(np.int64)

        def cast_all():
            import threading
            ths = [threading.Thread(target=oracle.cast, args=(FP32, E5M2, x[parts[t]:parts[t + 1]],
                                                               int(parts[t + 1] - parts[t]), 1.0, qs))
                   for t in range(threads)]
            for t in ths:
                t.start()
            for t in ths:
                t.join()
        out.append(line("cast_8192sq_fp32_e5m2", "cast 8192^2 FP32 -> E5M2 (scale, amax)", "GB/s", 1e-9,
                        "the whole 8192^2 cast", "port", lambda: oracle.cast(FP32, E5M2, x, n, 1.0, qs), cast_all,
                        n * 5))
        del x
    if "adam" in only:
        n = 256 * 1024 * 1024
        cfg = dict(lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, step=1, adamw=1,
                   bias_correction=1, grad_scale=1.0)
        for st, name, es in ((BF16, "bf16", 2), (FP32, "fp32", 4)):
            npd = np.uint16 if st == BF16 else np.float32
            p = np.full(n, 0.01, np.float32) if st == FP32 else np.full(n, 0x3C24, np.uint16)
            g = np.full(n, 1e-3, np.float32) if st == FP32 else np.full(n, 0x3A83, np.uint16)
            m, v = np.zeros(n, npd), np.zeros(n, npd)
            q = np.zeros(n, np.uint8)
            out.append(line(f"adamw_256m_{name}", f"adamw 256M params {name.upper()} p/g/m/v + E5M2 copy", "GB/s", 1e-9,
                            "one step over all 2^28 parameters", "port",
                            lambda: oracle.adam(cfg, st, p, st, g, st, m, v, E5M2, q, 1024.0, 0.0, threads=1),
                            lambda: oracle.adam(cfg, st, p, st, g, st, m, v, E5M2, q, 1024.0, 0.0, threads=threads),
                            n * (7 * es + 1)))
            del p, g, m, v, q
    return headline, out


def main():
    args = parse()
    if args.trace_summary:
        trace_summary(args.trace_summary, args.counters)
        return
    if args.traffic_json:
        traffic_json(*args.traffic_json)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from e5m2effma_amd import _lib

    L = _lib.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    only = set(args.only.split(","))
    K, W = args.steps, args.warmup
    keep = []

    def check(s, what):
        if s != 0:
            raise RuntimeError(f"{what}: {_lib.status_string(s)}: {_lib.last_error()}")

    def f32(v):
        t = torch.tensor([v], dtype=torch.float32, device=dev)
        keep.append(t)
        return t.data_ptr()

    def quantize(x, fmt, scale=1.0):
        """FP32 device tensor -> FP8 codes through e5ma_cast (RNE, satfinite)."""
        out = torch.empty(x.numel(), dtype=torch.uint8, device=dev)
        S = _lib.tensor(x.data_ptr(), FP32)
        D = _lib.tensor(out.data_ptr(), fmt, None, f32(scale) if scale != 1.0 else None)
        check(L.e5ma_cast(ctypes.byref(S), ctypes.byref(D), x.numel(), sp), "cast")
        return out

    def settle(fn, seconds):
        """Calls fn until `seconds` of wall time have passed (synchronizing every 8 calls): under FP8
        matrix load the clock takes ~20 ms to come down from its idle boost and settle, so a fixed small
        number of warm-up calls can leave the first timed calls on a clock still moving."""
        t0, calls = time.perf_counter(), 0
        while True:
            fn()
            calls += 1
            if calls % 8 == 0:
                torch.cuda.synchronize()
                if time.perf_counter() - t0 >= seconds:
                    return calls

    def timed(fn, steps, warmup):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(steps):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps  # ms per call

    def graph_timed(fn, calls, reps=3):
        """ms per call of `calls` back-to-back calls recorded in one HIP graph (fn(i, stream pointer)): the
        GPU-side rate without the host's per-call issue cost; median of `reps` replays."""
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            ssp = ctypes.c_void_p(side.cuda_stream)
            for i in range(calls):
                fn(i, ssp)
        graph.replay()
        torch.cuda.synchronize()
        res = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            graph.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            res.append(e0.elapsed_time(e1) / calls)
        del graph
        return sorted(res)[len(res) // 2]

    out = {}
    secondary = []
    g = torch.Generator(device=dev)
    traffic = traffic_table()

    def roof(bound, achieved, peak, unit, wid):
        return {"bound": bound, "achieved": round(achieved, 1), "peak": peak, "unit": unit,
                "frac": round(achieved / peak, 4), "traffic": traffic.get(wid)}

    # ---- GEMM 8192^3 ------------------------------------------------------------------------------
    if "gemm" in only:
        M = N = Kd = 8192
        g.manual_seed(0xE5A003)
        xa = torch.randn(M * Kd, device=dev, generator=g) * 8
        xb = torch.randn(N * Kd, device=dev, generator=g) * 8
        sat = torch.randint(0, M * Kd, (M * Kd // 10000,), device=dev, generator=g)
        xa[sat] = 57344.0
        xb[sat] = 57344.0
        A8 = quantize(xa, E5M2)
        B8 = {E4M3: quantize(xb, E4M3), E5M2: quantize(xb, E5M2)}
        Bbf = xb.to(torch.bfloat16)
        del xa, xb
        D = torch.empty(M * N, dtype=torch.bfloat16, device=dev)
        sinv = f32(1.0 / 64)
        flop = 2.0 * M * N * Kd

        def gemm_fn(bdt):
            Bdata = B8[bdt] if bdt != BF16 else Bbf
            At = _lib.tensor(A8.data_ptr(), E5M2, sinv)
            Bt = _lib.tensor(Bdata.data_ptr(), bdt, sinv if bdt != BF16 else None)
            Dt = _lib.tensor(D.data_ptr(), BF16)

            def f(i=0):
                check(L.e5ma_gemm(1, 0, M, N, Kd, 1.0, ctypes.byref(At), Kd, ctypes.byref(Bt), Kd, 0.0, None, 0,
                                  ctypes.byref(Dt), M, None, sp), "gemm")
            return f
        settle_calls = settle(gemm_fn(E4M3), SETTLE_S)
        ms = timed(gemm_fn(E4M3), K, W)
        tf = flop / (ms * 1e-3) / 1e12
        out["gemm"] = dict(ms=ms, tflops=tf, settle_calls=settle_calls)
        for bdt, name, peak in ((E5M2, "E5M2xE5M2", FP8_PEAK_TFLOPS), (BF16, "E5M2xBF16", BF16_PEAK_TFLOPS)):
            settle(gemm_fn(bdt), SETTLE_2ND_S)
            ms2 = timed(gemm_fn(bdt), max(3, K), 2)
            t2 = flop / (ms2 * 1e-3) / 1e12
            secondary.append({"workload": f"gemm 8192^3 {name}->BF16 TN", "id": f"gemm_8192_{name.lower()}",
                              "value": round(t2, 1), "unit": "TFLOP/s", "ms_per_call": round(ms2, 4),
                              "roofline": roof("mfma", t2, peak, "TFLOP/s", f"gemm_8192_{name.lower()}")})

        # the other three layouts of the headline GEMM (the same bytes read as M / N-contiguous operands)
        def layout_fn(ta, tb):
            At = _lib.tensor(A8.data_ptr(), E5M2, sinv)
            Bt = _lib.tensor(B8[E4M3].data_ptr(), E4M3, sinv)
            Dt = _lib.tensor(D.data_ptr(), BF16)

            def f(i=0):
                check(L.e5ma_gemm(ta, tb, M, N, Kd, 1.0, ctypes.byref(At), Kd if ta else M, ctypes.byref(Bt),
                                  N if tb else Kd, 0.0, None, 0, ctypes.byref(Dt), M, None, sp), "gemm")
            return f
        for ta, tb, lname in ((0, 0, "NN"), (0, 1, "NT"), (1, 1, "TT")):
            settle(layout_fn(ta, tb), SETTLE_2ND_S)
            ms2 = timed(layout_fn(ta, tb), max(3, K), 2)
            t2 = flop / (ms2 * 1e-3) / 1e12
            secondary.append({"workload": f"gemm 8192^3 E5M2xE4M3->BF16 {lname}", "id": f"gemm_8192_{lname.lower()}",
                              "value": round(t2, 1), "unit": "TFLOP/s", "ms_per_call": round(ms2, 4),
                              "roofline": roof("mfma", t2, FP8_PEAK_TFLOPS, "TFLOP/s", f"gemm_8192_{lname.lower()}")})
        del A8, B8, Bbf, D

    # ---- config 4: TE HYBRID backward GEMMs, tokens 8192, hidden 4096, ffn 14336 ----------------------
    progress("gemm lines done")
    if "te" in only:
        tok, hid, ffn = 8192, 4096, 14336
        g.manual_seed(0xE5A004 + 1)
        Wq = quantize(torch.randn(ffn * hid, device=dev, generator=g) * (0.02 * 64), E4M3)  # [ffn, hid] row-major
        dY = quantize(torch.randn(tok * ffn, device=dev, generator=g) * (1e-3 * 1024), E5M2)  # [tok, ffn] row-major
        X = quantize(torch.randn(tok * hid, device=dev, generator=g) * 2.0, E4M3)            # [tok, hid] row-major
        sw = torch.full((hid,), 1 / 64, device=dev)     # row-wise scale_inv of W^T (m = hid)
        sdy = torch.full((tok,), 1 / 1024, device=dev)  # row-wise scale_inv of dY (n = tok)
        dX = torch.empty(hid * tok, dtype=torch.bfloat16, device=dev)
        G = torch.zeros(ffn * hid, dtype=torch.float32, device=dev)
        bias = torch.zeros(ffn, dtype=torch.float32, device=dev)
        dX8 = torch.empty(hid * tok, dtype=torch.uint8, device=dev)
        am = torch.zeros(1, dtype=torch.float32, device=dev)
        dY_bad = dY.clone()
        hit = torch.randint(0, dY_bad.numel(), (dY_bad.numel() // 100000,), device=dev, generator=g)
        dY_bad[hit] = 0x7E  # E5M2 NaN codes (0.001 %)
        Wt = _lib.tensor(Wq.data_ptr(), E4M3, sw.data_ptr(), None, None, 1)
        dYt = _lib.tensor(dY.data_ptr(), E5M2, sdy.data_ptr(), None, None, 1)
        dYb = _lib.tensor(dY_bad.data_ptr(), E5M2, sdy.data_ptr(), None, None, 1)
        dYw = _lib.tensor(dY.data_ptr(), E5M2, f32(1 / 1024))
        Xt = _lib.tensor(X.data_ptr(), E4M3, f32(0.5))
        dXt = _lib.tensor(dX.data_ptr(), BF16)
        dX8t = _lib.tensor(dX8.data_ptr(), E5M2, None, f32(4.0), am.data_ptr())
        Gt = _lib.tensor(G.data_ptr(), FP32)
        Bt = _lib.tensor(bias.data_ptr(), FP32)

        # dgrad: dX^T [hid, tok] = W^T dY^T, column-major: e5ma_gemm(N, N, hid, tok, ffn), A = W (lda = hid),
        # B = dY (ldb = ffn), OUTER scale_inv vectors on both
        def dgrad(i=0, Bd=dYt, Dd=dXt):
            check(L.e5ma_gemm(0, 0, hid, tok, ffn, 1.0, ctypes.byref(Wt), hid, ctypes.byref(Bd), ffn, 0.0, None, 0,
                              ctypes.byref(Dd), hid, None, sp), "dgrad")

        # wgrad: main_grad [ffn, hid] (column-major ffn x hid) += dY^T X + bias: e5ma_gemm(N, T, ffn, hid, tok),
        # A = dY (lda = ffn), B = X (ldb = hid), beta = 1, C = NULL
        def wgrad(i=0):
            check(L.e5ma_gemm(0, 1, ffn, hid, tok, 1.0, ctypes.byref(dYw), ffn, ctypes.byref(Xt), hid, 1.0, None, 0,
                              ctypes.byref(Gt), ffn, ctypes.byref(Bt), sp), "wgrad")

        def dgrad8(i=0):
            dgrad(i, dYb, dX8t)

        # wgrad from token-contiguous FP8 copies (TE's transposed caches): main_grad^T [hid, ffn] += X^T dY,
        # e5ma_gemm(T, N, hid, ffn, tok), A = X^T storage [hid][tok], B = dY^T storage [ffn][tok]; the
        # bytes of X and dY stand in for the transposed copies (the kernel time does not depend on values)
        Gt2 = _lib.tensor(G.data_ptr(), FP32)
        bias2 = torch.zeros(hid, dtype=torch.float32, device=dev)
        Bt2 = _lib.tensor(bias2.data_ptr(), FP32)
        Xw = _lib.tensor(X.data_ptr(), E4M3, f32(0.5))

        def wgrad_tn(i=0):
            check(L.e5ma_gemm(1, 0, hid, ffn, tok, 1.0, ctypes.byref(Xw), tok, ctypes.byref(dYw), tok, 1.0, None, 0,
                              ctypes.byref(Gt2), hid, ctypes.byref(Bt2), sp), "wgrad_tn")
        flop = 2.0 * hid * tok * ffn
        for name, wid, fn in (("dgrad (N,N) E4M3 W x E5M2 dY, row-wise scale_inv, BF16 out", "te_dgrad", dgrad),
                              ("wgrad (N,T) E5M2 dY x E4M3 X, beta=1 into FP32 main_grad + bias", "te_wgrad", wgrad),
                              ("wgrad (T,N) from token-contiguous copies, beta=1 into FP32 + bias", "te_wgrad_tn",
                               wgrad_tn),
                              ("dgrad (N,N) E5M2 out, scale + amax, 0.001% NaN codes in dY", "te_dgrad_e5m2", dgrad8)):
            settle(fn, SETTLE_2ND_S)
            ms = timed(fn, max(3, K), max(W, 3))
            tf = flop / (ms * 1e-3) / 1e12
            secondary.append({"workload": f"TE config 4 {name}", "id": wid, "value": round(tf, 1), "unit": "TFLOP/s",
                              "ms_per_call": round(ms, 4),
                              "roofline": roof("mfma", tf, FP8_PEAK_TFLOPS, "TFLOP/s", wid)})
        del Wq, dY, X, dX, G, dX8, dY_bad, bias2

    # ---- GEMV 8192^2, batch 1 and 8 -----------------------------------------------------------------
    progress("te lines done")
    if "gemv" in only:
        M = Kd = 8192
        nbuf = 6
        g.manual_seed(0xE5A002)
        Ws, sas = [], []
        for b in range(nbuf):
            w = torch.randn(M * Kd, device=dev, generator=g) * 0.02
            amax = w.abs().max().item()
            Ws.append(quantize(w, E5M2, 57344.0 / amax))
            sas.append(torch.full((M,), amax / 57344.0, dtype=torch.float32, device=dev))
            del w
        for n in (1, 8):
            x = torch.randn(Kd * n, device=dev, generator=g).to(torch.bfloat16)
            y = torch.empty(M * n, dtype=torch.bfloat16, device=dev)
            descs = [(_lib.tensor(Ws[b].data_ptr(), E5M2, sas[b].data_ptr(), None, None, 1)) for b in range(nbuf)]
            Bt = _lib.tensor(x.data_ptr(), BF16)
            Dt = _lib.tensor(y.data_ptr(), BF16)

            def f(i=0, s=sp):
                check(L.e5ma_gemm(1, 0, M, n, Kd, 1.0, ctypes.byref(descs[i % nbuf]), Kd, ctypes.byref(Bt), Kd, 0.0,
                                  None, 0, ctypes.byref(Dt), M, None, s), "gemv")
            ms = timed(f, max(K, 30), W)
            # the same calls issued from a graph: a call here is shorter than the host's cost of issuing it
            # through ctypes, so the eager rate can be the host's
            msg = graph_timed(f, 120)
            nbytes = M * Kd + M * 4 + Kd * n * 2 + M * n * 2  # weights, row scales, x, y
            gbs = nbytes / (ms * 1e-3) / 1e9
            secondary.append({"workload": f"gemv 8192x8192 E5M2 (row-wise scale_inv) x BF16 n={n} -> BF16",
                              "id": f"gemv_8192_n{n}", "value": round(gbs, 1), "unit": "GB/s",
                              "ms_per_call": round(ms, 5), "bytes_per_call": nbytes,
                              "graph_ms_per_call": round(msg, 5),
                              "graph_frac": round(nbytes / (msg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                              "roofline": roof("hbm", gbs, HBM_PEAK_GBS, "GB/s", f"gemv_8192_n{n}")})
        del Ws, sas

        # the same kernel's streaming rate: 8x the rows (512 MiB of weights, two buffers rotated past the
        # Infinity Cache), where the per-call fixed cost (launch gap, ramp-up, tail) weighs 8x less
        M8 = 8 * M
        Wb = [torch.randint(0, 0x7B, (M8 * Kd,), dtype=torch.uint8, device=dev, generator=g) for _ in range(2)]
        sa8 = torch.full((M8,), 1.0 / 64, dtype=torch.float32, device=dev)
        x = torch.randn(Kd, device=dev, generator=g).to(torch.bfloat16)
        y = torch.empty(M8, dtype=torch.bfloat16, device=dev)
        descs = [_lib.tensor(w.data_ptr(), E5M2, sa8.data_ptr(), None, None, 1) for w in Wb]
        Bt, Dt = _lib.tensor(x.data_ptr(), BF16), _lib.tensor(y.data_ptr(), BF16)

        def f(i=0):
            check(L.e5ma_gemm(1, 0, M8, 1, Kd, 1.0, ctypes.byref(descs[i % 2]), Kd, ctypes.byref(Bt), Kd, 0.0, None, 0,
                              ctypes.byref(Dt), M8, None, sp), "gemv")
        ms = timed(f, max(K, 30), W)
        nbytes = M8 * Kd + M8 * 4 + Kd * 2 + M8 * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        secondary.append({"workload": "gemv 65536x8192 E5M2 x BF16 n=1 -> BF16 (streaming rate of the n=1 kernel)",
                          "id": "gemv_65536x8192_n1", "value": round(gbs, 1), "unit": "GB/s",
                          "ms_per_call": round(ms, 5), "bytes_per_call": nbytes,
                          "roofline": roof("hbm", gbs, HBM_PEAK_GBS, "GB/s", "gemv_65536x8192_n1")})
        del Wb

    # ---- AdamW 256M parameters ----------------------------------------------------------------------
    progress("gemv lines done")
    if "adam" in only:
        n = 256 * 1024 * 1024
        for st, name in ((BF16, "BF16"), (FP32, "FP32")):
            tdt = torch.bfloat16 if st == BF16 else torch.float32
            g.manual_seed(0xE5A005)
            p = (torch.randn(n, device=dev, generator=g) * 0.02).to(tdt)
            gr = (torch.randn(n, device=dev, generator=g) * 1e-3).to(tdt)
            m = torch.zeros(n, dtype=tdt, device=dev)
            v = torch.zeros(n, dtype=tdt, device=dev)
            q = torch.empty(n, dtype=torch.uint8, device=dev)
            am = torch.zeros(1, dtype=torch.float32, device=dev)
            qs = f32(57344.0 / 0.1)
            P, G, Mo, V = (_lib.tensor(t.data_ptr(), st) for t in (p, gr, m, v))
            Q = _lib.tensor(q.data_ptr(), E5M2, None, qs, am.data_ptr())
            step = [0]

            def f(i=0):
                step[0] += 1
                cfg = _lib.AdamConfig(1e-4, 0.9, 0.999, 1e-8, 0.01, step[0], 1, 1, 1.0)
                check(L.e5ma_adam(ctypes.byref(cfg), n, ctypes.byref(P), ctypes.byref(G), ctypes.byref(Mo),
                                  ctypes.byref(V), ctypes.byref(Q), sp), "adam")
            ms = timed(f, 10, 2)
            es = 2 if st == BF16 else 4
            nbytes = n * (7 * es + 1)  # read p, g, m, v; write p, m, v; write the FP8 copy
            gbs = nbytes / (ms * 1e-3) / 1e9
            secondary.append({"workload": f"adamw 256M params {name} p/g/m/v + E5M2 copy",
                              "id": f"adamw_256m_{name.lower()}", "value": round(gbs, 1), "unit": "GB/s",
                              "ms_per_call": round(ms, 4), "bytes_per_call": nbytes,
                              "roofline": roof("hbm", gbs, HBM_PEAK_GBS, "GB/s", f"adamw_256m_{name.lower()}")})
            del p, gr, m, v, q

    # ---- cast 8192^2 FP32 -> E5M2 --------------------------------------------------------------------
    progress("adam lines done")
    if "cast" in only:
        n = 8192 * 8192
        nbuf = 2  # 2 x 268 MB of sources rotate past the Infinity Cache
        g.manual_seed(0xE5A004)
        srcs = [torch.randn(n, device=dev, generator=g) * 0.02 for _ in range(nbuf)]
        dst = torch.empty(n, dtype=torch.uint8, device=dev)
        am = torch.zeros(1, dtype=torch.float32, device=dev)
        amax = srcs[0].abs().max().item()
        descs = [_lib.tensor(s.data_ptr(), FP32) for s in srcs]

        for fmt, fname, qmax in ((E5M2, "E5M2", 57344.0), (E4M3, "E4M3", 448.0)):
            Dt = _lib.tensor(dst.data_ptr(), fmt, None, f32(qmax / amax), am.data_ptr())

            def f(i=0, Dt=Dt):
                check(L.e5ma_cast(ctypes.byref(descs[i % nbuf]), ctypes.byref(Dt), n, sp), "cast")
            ms = timed(f, max(K, 20), W)
            nbytes = n * 5
            gbs = nbytes / (ms * 1e-3) / 1e9
            wid = f"cast_8192sq_fp32_{fname.lower()}"
            secondary.append({"workload": f"cast 8192x8192 FP32 -> {fname} (scale = {qmax:g} / amax, amax)", "id": wid,
                              "value": round(gbs, 1), "unit": "GB/s", "ms_per_call": round(ms, 5),
                              "bytes_per_call": nbytes, "roofline": roof("hbm", gbs, HBM_PEAK_GBS, "GB/s", wid)})

        # Float8Tensor.from_float's quantization in one e5ma_quantize call: per tensor, an amax pass then
        # the scaled cast (4 + 4 + 1 bytes per element); per row, each 8192-element row read once
        # (4 + 1 bytes per element, plus scale_inv and amax per row)
        qsc = torch.empty(8192, dtype=torch.float32, device=dev)
        qam = torch.empty(8192, dtype=torch.float32, device=dev)
        for wid, fmt, per_row, what in (
                ("quantize_8192sq_fp32_e5m2_tensor", E5M2, False, "per tensor: amax pass + scaled cast"),
                ("quantize_8192sq_fp32_e4m3_rows", E4M3, True, "per row, rows read once")):
            Dq = _lib.tensor(dst.data_ptr(), fmt, scaling=_lib.SCALING_OUTER if per_row else _lib.SCALING_TENSOR)
            rows, cols = (8192, 8192) if per_row else (1, n)

            def f(i=0, Dq=Dq, rows=rows, cols=cols):
                check(L.e5ma_quantize(ctypes.byref(descs[i % nbuf]), ctypes.byref(Dq), rows, cols,
                                      57344.0 if fmt == E5M2 else 448.0, qsc.data_ptr(), qam.data_ptr(), sp),
                      "quantize")
            ms = timed(f, max(K, 20), W)
            nbytes = n * 5 + 8192 * 8 if per_row else n * 9
            gbs = nbytes / (ms * 1e-3) / 1e9
            secondary.append({"workload": f"quantize 8192x8192 FP32 -> {'E4M3' if fmt == E4M3 else 'E5M2'} with "
                                          f"scale from amax ({what})", "id": wid,
                              "value": round(gbs, 1), "unit": "GB/s", "ms_per_call": round(ms, 5),
                              "bytes_per_call": nbytes, "roofline": roof("hbm", gbs, HBM_PEAK_GBS, "GB/s", wid)})
        del srcs, dst

    # ---- device copy 1 GiB: the practical streaming ceiling and the counters' calibration kernel -----
    progress("cast lines done")
    if "copy" in only:
        n = 256 * 1024 * 1024
        src = torch.randn(n, device=dev, generator=g)
        dsts = [torch.empty(n, device=dev) for _ in range(2)]

        def f(i=0):
            dsts[i % 2].copy_(src)
        ms = timed(f, max(K, 20), W)
        nbytes = n * 4 * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        secondary.append({"workload": "device copy 1 GiB FP32 (torch copy_), reference rate", "id": "copy_1gib",
                          "value": round(gbs, 1), "unit": "GB/s", "ms_per_call": round(ms, 4), "bytes_per_call": nbytes,
                          "roofline": roof("hbm", gbs, HBM_PEAK_GBS, "GB/s", "copy_1gib")})
        del src, dsts

    # ---- CPU baselines (the reference's CPU semantics, timed on this host's cores) ----------------------
    cpu, cpu_lines = None, []
    if not args.no_cpu:
        cpu, cpu_lines = cpu_baselines(only)

    res = {"metric": "FP8 GEMM TFLOP/s @8192^3 (% FP8 peak); GEMV + AdamW HBM GB/s (% of 8 TB/s)",
           "unit": "TFLOP/s", "n_gpus": 1, "steps": K, "warmup": W, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "fp8", "data": "synthetic"}
    if "gemm" in out:
        tf = out["gemm"]["tflops"]
        res.update({"value": round(tf, 1), "ms_per_step": round(out["gemm"]["ms"], 4),
                    "clock_settle": {"seconds": SETTLE_S, "calls": out["gemm"]["settle_calls"],
                                     "secondary_gemm_seconds": SETTLE_2ND_S,
                                     "note": "untimed headline calls before the W warm-up calls; each secondary "
                                             "GEMM line likewise, then K timed calls"},
                    "config": {"workload": "gemm 8192x8192x8192 E5M2 x E4M3 -> BF16, TN, scale_inv 1/64, alpha 1, "
                                           "beta 0 (BASELINE config 3 shape, north-star pairing)"},
                    "roofline": roof("mfma", tf, FP8_PEAK_TFLOPS, "TFLOP/s", "gemm_8192_e5m2xe4m3")})
    else:
        res.update({"value": None, "ms_per_step": None, "config": {"workload": "gemm not run (--only)"}})
    res["cpu_baseline"] = cpu
    res["cpu_baselines"] = cpu_lines
    res["secondary"] = secondary
    print(json.dumps(res))


if __name__ == "__main__":
    main()
