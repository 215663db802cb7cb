"""GPU-side helpers of the parity tests: run the C ABI on device buffers built from numpy arrays and
check the results with the CPU oracle (oracle/).  Shared by tests/, __graft_entry__.smoke() and
bench.py's checks; the product package never imports this."""
import ctypes

import numpy as np
import torch

import oracle
from e5m2effma_amd import _lib

NPD = oracle.NP_DTYPE
FP8 = (oracle.E5M2, oracle.E4M3)


def to_dev(arr, dev, offset=0):
    """A device copy of a numpy array as raw bytes; returns (holder tensor, device address).  offset
    shifts the data by that many bytes from a 256-byte aligned allocation (alignment tests)."""
    raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
    t = torch.empty(raw.size + offset + 16, dtype=torch.uint8, device=dev)
    t[offset:offset + raw.size].copy_(torch.from_numpy(raw))
    return t, t.data_ptr() + offset


def from_dev(t, addr, dtype, count):
    off = addr - t.data_ptr()
    nbytes = count * np.dtype(dtype).itemsize
    return t[off:off + nbytes].cpu().numpy().view(dtype).copy()


def dev_floats(vals, dev):
    t = torch.tensor(np.asarray(vals, np.float32).ravel(), dtype=torch.float32, device=dev)
    return t, t.data_ptr()


def finite_fp8(rng, n, fmt):
    """Finite FP8 codes uniformly over the code space, with the reference fixtures' rule for the
    Inf / NaN codes (tests/test_util.h:57-63): replaced by a finite neighbour."""
    c = rng.integers(0, 256, n).astype(np.uint8)
    bad = (c & 0x7C) == 0x7C if fmt == oracle.E5M2 else (c & 0x7F) == 0x7F
    c[bad] ^= 4 if fmt == oracle.E5M2 else 1
    return c


def normal_fp8(rng, n, fmt, sigma):
    """FP8 codes of N(0, sigma) values (RNE satfinite)."""
    return oracle.encode(fmt, rng.standard_normal(n).astype(np.float32) * np.float32(sigma))


def operand(rng, dt, size, dist="codes", sigma=1.0):
    if dt in FP8:
        return finite_fp8(rng, size, dt) if dist == "codes" else normal_fp8(rng, size, dt, sigma)
    x = (rng.uniform(-2, 2, size) if dist == "codes" else rng.standard_normal(size) * sigma).astype(np.float32)
    return oracle.encode(oracle.BF16, x) if dt == oracle.BF16 else x


class GemmCase:
    """One e5ma_gemm call: seeded operands, the GPU run through the C ABI, the oracle check.

    transa / transb: 1 = T.  sa / sb: None, a float (per tensor) or an array (OUTER scaling).  ldd / ldc:
    leading dimensions of D / C (default m + 3 / m + 5).
    beta != 0 with cdt None accumulates into D (C = NULL); otherwise C of dtype cdt is read."""

    def __init__(self, rng, transa, transb, m, n, k, adt, bdt, *, ddt=oracle.FP32, alpha=1.0, sa=None, sb=None,
                 beta=0.0, cdt=None, csinv=1.0, biasdt=None, qscale=None, amax=False, pad=16, dist="codes",
                 sigma=1.0, A=None, B=None, D0=None, ldd=None, ldc=None):
        self.transa, self.transb, self.m, self.n, self.k = transa, transb, m, n, k
        self.adt, self.bdt, self.ddt, self.alpha, self.beta = adt, bdt, ddt, alpha, beta
        self.lda = (k if transa else m) + pad
        self.ldb = (n if transb else k) + pad
        self.lda = (self.lda + 15) // 16 * 16
        self.ldb = (self.ldb + 15) // 16 * 16
        # default ldd = m + 3 (padding rows catch stray writes; not a multiple of 4, so the kernels take their
        # general epilogue); ldd = m + 4 with m % 4 == 0 keeps the padding and allows the direct epilogue
        self.ldd = ldd if ldd is not None else m + (3 if m > 1 else 0)
        self.A = A if A is not None else operand(rng, adt, self.lda * (m if transa else k), dist, sigma)
        self.B = B if B is not None else operand(rng, bdt, self.ldb * (k if transb else n), dist, sigma)
        self.sa, self.sb = sa, sb
        self.cdt, self.csinv = cdt, csinv
        self.C = None
        self.ldc = 0
        if beta != 0.0 and cdt is not None:
            self.ldc = ldc if ldc is not None else m + 5
            self.C = operand(rng, cdt, self.ldc * n) if cdt in FP8 else \
                oracle.encode(cdt, rng.uniform(-4, 4, self.ldc * n).astype(np.float32)) if cdt != oracle.FP32 else \
                rng.uniform(-4, 4, self.ldc * n).astype(np.float32)
        self.biasdt = biasdt
        self.bias = None
        if biasdt is not None:
            bv = rng.uniform(-8, 8, m).astype(np.float32)
            self.bias = bv if biasdt == oracle.FP32 else oracle.encode(biasdt, bv)
        self.qscale, self.amax = qscale, amax
        if D0 is not None:
            self.D0 = D0
        elif beta != 0.0 and cdt is None:  # accumulate into D: give it values
            v = rng.uniform(-4, 4, self.ldd * n).astype(np.float32)
            self.D0 = v if ddt == oracle.FP32 else oracle.encode(ddt, v, 1.0)
        else:  # 0xA5 fill catches stray or missing writes
            self.D0 = np.full(self.ldd * n * oracle.ESIZE[ddt], 0xA5, np.uint8).view(NPD[ddt]).copy()

    def oracle_gemm(self):
        g = oracle.Gemm(self.transa, self.transb, self.m, self.n, self.k, self.alpha, self.adt, self.A, self.lda,
                        self.bdt, self.B, self.ldb,
                        sa=None if self.sa is None else np.atleast_1d(np.float32(self.sa)),
                        sa_vec=self.sa is not None and np.ndim(self.sa) > 0,
                        sb=None if self.sb is None else np.atleast_1d(np.float32(self.sb)),
                        sb_vec=self.sb is not None and np.ndim(self.sb) > 0,
                        beta=self.beta, cdt=self.cdt, C=self.C, ldc=self.ldc, csinv=self.csinv, ddt=self.ddt,
                        D=self.D0.copy(), ldd=self.ldd, qscale=1.0 if self.qscale is None else self.qscale,
                        biasdt=self.biasdt if self.biasdt is not None else oracle.FP32, bias=self.bias,
                        ocp_operands=True)
        return g

    def workspace_bytes(self):
        """e5ma_gemm_workspace_size for this call on the current device."""
        return _lib.workspace_size(self.transa, self.transb, self.m, self.n, self.k, self.adt, self.lda, self.bdt,
                                   self.ldb)

    def run(self, dev, stream=None, workspace=None):
        """Run on the GPU; returns (status, D as numpy, amax or None).  workspace: None runs e5ma_gemm;
        a byte count runs e5ma_gemm_ex with a fresh device workspace of that size ("query": the size
        e5ma_gemm_workspace_size reports)."""
        keep = []

        def put(a):
            if a is None:
                return None
            t, p = to_dev(a, dev)
            keep.append(t)
            return p

        def scl(v):
            if v is None:
                return None, 0
            t, p = dev_floats(v, dev)
            keep.append(t)
            return p, int(np.ndim(v) > 0)
        pa, pb, pc, pbias = put(self.A), put(self.B), put(self.C), put(self.bias)
        Dt, pd = to_dev(self.D0, dev)
        sa_p, sa_o = scl(self.sa)
        sb_p, sb_o = scl(self.sb)
        cs_p, _ = scl(self.csinv if self.cdt in FP8 else None)
        q_p, _ = scl(self.qscale)
        am_t = torch.zeros(1, dtype=torch.float32, device=dev) if self.amax else None
        A = _lib.tensor(pa, self.adt, sa_p, None, None, sa_o)
        B = _lib.tensor(pb, self.bdt, sb_p, None, None, sb_o)
        C = _lib.tensor(pc, self.cdt, cs_p) if self.C is not None else None
        D = _lib.tensor(pd, self.ddt, None, q_p, None if am_t is None else am_t.data_ptr())
        bias = _lib.tensor(pbias, self.biasdt) if self.bias is not None else None
        st = ctypes.c_void_p(stream if stream is not None else torch.cuda.current_stream(dev).cuda_stream)
        L = _lib.lib()
        args = (self.transa, self.transb, self.m, self.n, self.k, float(self.alpha), _lib.ref(A), self.lda,
                _lib.ref(B), self.ldb, float(self.beta), _lib.ref(C), self.ldc, _lib.ref(D), self.ldd, _lib.ref(bias))
        if workspace is None:
            s = L.e5ma_gemm(*args, st)
        else:
            nbytes = self.workspace_bytes() if workspace == "query" else int(workspace)
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
            keep.append(ws)
            s = L.e5ma_gemm_ex(*args, ws.data_ptr() if nbytes else None, nbytes, st)
        torch.cuda.synchronize(dev)
        D_got = from_dev(Dt, pd, NPD[self.ddt], self.ldd * self.n)
        return s, D_got, (None if am_t is None else float(am_t.item()))

    def check(self, D_got, amax=None, samples=None, rng=None, err_factor=2.0):
        """(bad count, first bad index) of the oracle bound over all outputs (or `samples` random ones);
        also the padding rows of D must be untouched and amax inside the oracle's interval."""
        g = self.oracle_gemm()
        if samples is None:
            iis, jjs = [a.ravel() for a in np.meshgrid(np.arange(self.m), np.arange(self.n), indexing="ij")]
        else:
            iis = rng.integers(0, self.m, samples)
            jjs = rng.integers(0, self.n, samples)
        C_before = self.C if self.C is not None else (self.D0 if self.beta != 0.0 else None)
        bad, first, alo, ahi = g.check(D_got, C_before, iis, jjs, err_factor=err_factor)
        if self.ldd > self.m:  # rows m .. ldd-1 of every column are padding
            pad = np.concatenate([D_got.reshape(self.n, self.ldd)[:, self.m:].view(np.uint8).ravel()])
            ref = np.concatenate([self.D0.reshape(self.n, self.ldd)[:, self.m:].view(np.uint8).ravel()])
            assert np.array_equal(pad, ref), "stray writes into the ldd padding of D"
        if amax is not None and samples is None:
            assert alo <= amax <= ahi or (alo == ahi == amax), (amax, alo, ahi)
        return bad, first

    def run_and_check(self, dev, **kw):
        s, D, amax = self.run(dev)
        assert s == 0, (s, _lib.last_error())
        return self.check(D, amax, **kw)


def gpu_cast(dev, tin, tout, x, sinv=None, qscale=None, amax0=0.0, offset_in=0, offset_out=0, want_amax=True):
    """e5ma_cast of numpy array x (dtype NPD[tin]); returns (result array, amax or None)."""
    keep = []
    xt, px = to_dev(np.ascontiguousarray(x, NPD[tin]), dev, offset_in)
    n = x.size
    out = torch.empty(n * oracle.ESIZE[tout] + offset_out + 16, dtype=torch.uint8, device=dev)
    po = out.data_ptr() + offset_out
    sp = qp = None
    if sinv is not None:
        t, sp = dev_floats(sinv, dev)
        keep.append(t)
    if qscale is not None:
        t, qp = dev_floats(qscale, dev)
        keep.append(t)
    am = torch.full((1,), amax0, dtype=torch.float32, device=dev) if want_amax else None
    S = _lib.tensor(px, tin, sp)
    D = _lib.tensor(po, tout, None, qp, None if am is None else am.data_ptr())
    s = _lib.lib().e5ma_cast(ctypes.byref(S), ctypes.byref(D), n, ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    assert s == 0, (s, _lib.last_error())
    torch.cuda.synchronize(dev)
    res = from_dev(out, po, NPD[tout], n)
    return res, (None if am is None else float(am.item()))


def _state_values(rng, dt, n, scale, positive=False):
    v = rng.standard_normal(n).astype(np.float32) * np.float32(scale)
    if positive:
        v = np.abs(v)
    return v if dt == oracle.FP32 else oracle.encode(dt, v)


def adam_matches(dev, rng, n, pdt, gdt, mdt, qdt=None, steps=3, offset=0, cfg=None, qscale=64.0):
    """Runs `steps` Adam steps on the GPU (C ABI) and in the oracle from the same state; True when
    param, exp_avg, exp_avg_sq, the FP8 copy and amax agree bit for bit after every step."""
    cfg = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, adamw=1, bias_correction=1,
               grad_scale=0.5) if cfg is None else dict(cfg)
    p = _state_values(rng, pdt, n, 0.02 * 50)
    m = _state_values(rng, mdt, n, 1e-3)
    v = _state_values(rng, mdt, n, 1e-6, positive=True)
    pt, pp = to_dev(p, dev, offset * oracle.ESIZE[pdt])
    mt, pm = to_dev(m, dev, offset * oracle.ESIZE[mdt])
    vt, pv = to_dev(v, dev, offset * oracle.ESIZE[mdt])
    keep = []
    qt = qp = amt = qs_t = None
    q_np = None
    if qdt is not None:
        q_np = np.zeros(n, np.uint8)
        qt, qp = to_dev(q_np, dev, offset)
        amt = torch.zeros(1, dtype=torch.float32, device=dev)
        qs_t, _ = dev_floats(qscale, dev)
    amax_ref = 0.0
    for step in range(1, steps + 1):
        g = _state_values(rng, gdt, n, 1e-3)
        gt, pg = to_dev(g, dev, offset * oracle.ESIZE[gdt])
        keep.append(gt)
        c = dict(cfg, step=step)
        C = _lib.AdamConfig(c["lr"], c["beta1"], c["beta2"], c["eps"], c["weight_decay"], step, c["adamw"],
                            c["bias_correction"], c["grad_scale"])
        P, G = _lib.tensor(pp, pdt), _lib.tensor(pg, gdt)
        Mo, V = _lib.tensor(pm, mdt), _lib.tensor(pv, mdt)
        Q = _lib.tensor(qp, qdt, None, qs_t.data_ptr(), amt.data_ptr()) if qdt is not None else None
        s = _lib.lib().e5ma_adam(ctypes.byref(C), n, ctypes.byref(P), ctypes.byref(G), ctypes.byref(Mo),
                                 ctypes.byref(V), _lib.ref(Q), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
        assert s == 0, (s, _lib.last_error())
        amax_ref = oracle.adam(c, pdt, p, gdt, g, mdt, m, v, qdt if qdt is not None else oracle.E4M3, q_np,
                               qscale, amax_ref, threads=8)
        torch.cuda.synchronize(dev)
        gp = from_dev(pt, pp, NPD[pdt], n)
        gm = from_dev(mt, pm, NPD[mdt], n)
        gv = from_dev(vt, pv, NPD[mdt], n)
        for name, a, b in (("param", gp, p), ("exp_avg", gm, m), ("exp_avg_sq", gv, v)):
            if not np.array_equal(a.view(np.uint8), b.view(np.uint8)):
                bad = np.nonzero(a.view(np.uint8) != b.view(np.uint8))[0]
                print(f"adam step {step}: {name} differs at {bad.size} bytes, first {bad[:4]}")
                return False
        if qdt is not None:
            gq = from_dev(qt, qp, np.uint8, n)
            if not np.array_equal(gq, q_np):
                print(f"adam step {step}: FP8 copy differs at {np.count_nonzero(gq != q_np)} elements")
                return False
            if np.float32(amt.item()) != np.float32(amax_ref):
                print(f"adam step {step}: amax {amt.item()} != {amax_ref}")
                return False
    return True
