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
    return p.parse_args()


def main():
    args = parse()
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
            ms2 = timed(gemm_fn(bdt), max(3, K // 2), 2)
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
            ms2 = timed(layout_fn(ta, tb), max(3, K // 2), 2)
            t2 = flop / (ms2 * 1e-3) / 1e12
            secondary.append({"workload": f"gemm 8192^3 E5M2xE4M3->BF16 {lname}", "id": f"gemm_8192_{lname.lower()}",
                              "value": round(t2, 1), "unit": "TFLOP/s", "ms_per_call": round(ms2, 4),
                              "roofline": roof("mfma", t2, FP8_PEAK_TFLOPS, "TFLOP/s", f"gemm_8192_{lname.lower()}")})
        del A8, B8, Bbf, D

    # ---- config 4: TE HYBRID backward GEMMs, tokens 8192, hidden 4096, ffn 14336 ----------------------
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
            ms = timed(fn, max(3, K // 2), max(W, 3))
            tf = flop / (ms * 1e-3) / 1e12
            secondary.append({"workload": f"TE config 4 {name}", "id": wid, "value": round(tf, 1), "unit": "TFLOP/s",
                              "ms_per_call": round(ms, 4),
                              "roofline": roof("mfma", tf, FP8_PEAK_TFLOPS, "TFLOP/s", wid)})
        del Wq, dY, X, dX, G, dX8, dY_bad, bias2

    # ---- GEMV 8192^2, batch 1 and 8 -----------------------------------------------------------------
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

            def f(i=0):
                check(L.e5ma_gemm(1, 0, M, n, Kd, 1.0, ctypes.byref(descs[i % nbuf]), Kd, ctypes.byref(Bt), Kd, 0.0,
                                  None, 0, ctypes.byref(Dt), M, None, sp), "gemv")
            ms = timed(f, max(K, 30), W)
            nbytes = M * Kd + M * 4 + Kd * n * 2 + M * n * 2  # weights, row scales, x, y
            gbs = nbytes / (ms * 1e-3) / 1e9
            secondary.append({"workload": f"gemv 8192x8192 E5M2 (row-wise scale_inv) x BF16 n={n} -> BF16",
                              "id": f"gemv_8192_n{n}", "value": round(gbs, 1), "unit": "GB/s",
                              "ms_per_call": round(ms, 5), "bytes_per_call": nbytes,
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
    if "cast" in only:
        n = 8192 * 8192
        nbuf = 2  # 2 x 268 MB of sources rotate past the Infinity Cache
        g.manual_seed(0xE5A004)
        srcs = [torch.randn(n, device=dev, generator=g) * 0.02 for _ in range(nbuf)]
        dst = torch.empty(n, dtype=torch.uint8, device=dev)
        am = torch.zeros(1, dtype=torch.float32, device=dev)
        amax = srcs[0].abs().max().item()
        descs = [_lib.tensor(s.data_ptr(), FP32) for s in srcs]
        Dt = _lib.tensor(dst.data_ptr(), E5M2, None, f32(57344.0 / amax), am.data_ptr())

        def f(i=0):
            check(L.e5ma_cast(ctypes.byref(descs[i % nbuf]), ctypes.byref(Dt), n, sp), "cast")
        ms = timed(f, max(K, 20), W)
        nbytes = n * 5
        gbs = nbytes / (ms * 1e-3) / 1e9
        secondary.append({"workload": "cast 8192x8192 FP32 -> E5M2 (scale, amax)", "id": "cast_8192sq_fp32_e5m2",
                          "value": round(gbs, 1), "unit": "GB/s", "ms_per_call": round(ms, 5), "bytes_per_call": nbytes,
                          "roofline": roof("hbm", gbs, HBM_PEAK_GBS, "GB/s", "cast_8192sq_fp32_e5m2")})

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

    # ---- CPU baseline: the oracle's FFMA chain on a slab of the 8192^3 GEMM ---------------------------
    cpu = None
    if not args.no_cpu and "gemm" in only:
        import numpy as np
        import oracle
        rng = np.random.default_rng(1)
        Md = Nd = Kd = 8192
        A = oracle.encode(E5M2, (rng.standard_normal(Kd * 64) * 8).astype(np.float32))
        A = np.tile(A, Md // 64)  # the chain's cost does not depend on the values
        B = oracle.encode(E4M3, (rng.standard_normal(Kd * 64) * 8).astype(np.float32))
        B = np.tile(B, Nd // 64)
        threads = max(1, min(16, os.cpu_count() or 1))
        gm = oracle.Gemm(1, 0, Md, Nd, Kd, 1.0, E5M2, A, Kd, E4M3, B, Kd, sa=[1 / 64], sb=[1 / 64], ddt=BF16)
        rows = 2
        while True:
            t0 = time.perf_counter()
            gm.chain(rows=(0, rows), threads=threads)
            dt = time.perf_counter() - t0
            if dt > 2.0 or rows >= 64:
                break
            rows *= 2
        cpu_tflops = 2.0 * rows * Nd * Kd / dt / 1e12
        cpu = {"value": round(cpu_tflops, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
               "sample": f"{rows} of 8192 output rows of the 8192^3 E5M2 x E4M3 GEMM, ascending-k FP32 fmaf chain "
                         f"(oracle/e5ma_oracle.c, {threads} threads), rate scaled to the full problem"}

    res = {"metric": "FP8 GEMM TFLOP/s @8192^3 (% FP8 peak); GEMV + AdamW HBM GB/s (% of 8 TB/s)",
           "unit": "TFLOP/s", "n_gpus": 1, "steps": K, "warmup": W, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "fp8", "data": "synthetic"}
    if "gemm" in out:
        tf = out["gemm"]["tflops"]
        res.update({"value": round(tf, 1), "ms_per_step": round(out["gemm"]["ms"], 4),
                    "clock_settle": {"seconds": SETTLE_S, "calls": out["gemm"]["settle_calls"],
                                     "note": "untimed headline calls before the W warm-up calls"},
                    "config": {"workload": "gemm 8192x8192x8192 E5M2 x E4M3 -> BF16, TN, scale_inv 1/64, alpha 1, "
                                           "beta 0 (BASELINE config 3 shape, north-star pairing)"},
                    "roofline": roof("mfma", tf, FP8_PEAK_TFLOPS, "TFLOP/s", "gemm_8192_e5m2xe4m3")})
    else:
        res.update({"value": None, "ms_per_step": None, "config": {"workload": "gemm not run (--only)"}})
    res["cpu_baseline"] = cpu
    res["secondary"] = secondary
    print(json.dumps(res))


if __name__ == "__main__":
    main()
