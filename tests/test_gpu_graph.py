"""The C ABI under HIP graph capture.  The entry points allocate nothing, record no memset nodes and never
synchronize, so a caller can record them into a graph: here one graph holds a per-tensor and a per-row
quantize, FP8 GEMMs on the FP8 matrix cores (BF16 output with bias; E5M2 output with scale and amax), a
BF16-matrix-core GEMM accumulating into an FP32 D, split-K GEMMs through e5ma_gemm_ex and
e5ma_gemm_noalloc, GEMVs at n = 1 and n = 8, a cast with amax and an AdamW step with an FP8 copy.

The graph is replayed several times.  Before each replay the host resets the state the calls update in
place (the accumulated D, the Adam state, the max-reduced amax words) and fills every output with a
0xA5 pattern; between replays it runs eager work of its own and synchronizes.  Every replay's outputs
must equal those of the same calls issued eagerly, bit for bit.  The eager results themselves are held
to the oracle by the other GPU tests; here a few are checked again (per-tensor quantize, GEMV n = 1)."""
import ctypes

import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle
from e5m2effma_amd import _lib

pytestmark = pytest.mark.gpu
E5, E4, B16, F32 = oracle.E5M2, oracle.E4M3, oracle.BF16, oracle.FP32
K = 8192


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


class Calls:
    """Device buffers of the recorded calls and the calls themselves (issue(stream))."""

    def __init__(self, dev, rng):
        f32 = lambda *s: torch.empty(*s, dtype=torch.float32, device=dev)
        u8 = lambda n: torch.empty(n, dtype=torch.uint8, device=dev)
        u16 = lambda n: torch.empty(n, dtype=torch.int16, device=dev)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        self.dev = dev
        # inputs (never written by the calls)
        self.X = t(rng.standard_normal((512, K)).astype(np.float32) * 3)
        self.W = t(rng.standard_normal((1024, K)).astype(np.float32) * 0.05)
        self.bias16 = t(oracle.encode(B16, rng.uniform(-1, 1, 1024).astype(np.float32)).view(np.int16))
        self.bias32 = t(rng.uniform(-1, 1, 512).astype(np.float32))
        self.x1 = t(oracle.encode(B16, rng.uniform(-1, 1, K).astype(np.float32)).view(np.int16))
        self.x8 = t(oracle.encode(B16, rng.uniform(-1, 1, 8 * K).astype(np.float32)).view(np.int16))
        self.Xc = t(rng.standard_normal(1 << 20).astype(np.float32) * 100)
        self.G = t(rng.standard_normal((1 << 20) + 3).astype(np.float32) * 1e-3)
        self.q2 = t(np.float32([0.5]))
        self.qc = t(np.float32([4.0]))
        self.qa = t(np.float32([64.0]))
        # state updated in place, with its initial contents
        self.init = {
            "D3": t(rng.uniform(-4, 4, 512 * 1024).astype(np.float32)),
            "P": t(oracle.encode(B16, rng.standard_normal((1 << 20) + 3).astype(np.float32)).view(np.int16)),
            "M": t(rng.standard_normal((1 << 20) + 3).astype(np.float32) * 1e-3),
            "V": t(np.abs(rng.standard_normal((1 << 20) + 3)).astype(np.float32) * 1e-6),
        }
        self.state = {k: v.clone() for k, v in self.init.items()}
        self.amax = {k: f32(1) for k in ("a2", "ac", "aa")}
        # outputs
        self.out = {
            "Xq": u8(512 * K), "sx": f32(1), "ax": f32(1),
            "Wq": u8(1024 * K), "sw": f32(1024), "aw": f32(1024),
            "D1": u16(512 * 1024), "D2": u8(512 * 1024), "D4": f32(512 * 512), "D5": f32(512 * 512),
            "D6": f32(1024), "D7": u16(8 * 1024), "Cc": u8(1 << 20), "Q": u8((1 << 20) + 3),
        }
        nbytes = _lib.workspace_size(_lib.OP_T, _lib.OP_N, 512, 512, K, E5, K, E4, K)
        assert nbytes > 0, "a 4-tile GEMM splits K when given a workspace"
        self.ws = u8(nbytes)
        self.ws_bytes = nbytes

    def reset(self):
        """Eager: in-place state back to its initial contents, amax words to 0, outputs to 0xA5."""
        for k, v in self.state.items():
            v.copy_(self.init[k])
        for v in self.amax.values():
            v.zero_()
        for v in self.out.values():
            v.view(torch.uint8).fill_(0xA5)

    def snapshot(self):
        items = list(self.out.items()) + list(self.amax.items()) + list(self.state.items())
        return {k: v.view(torch.uint8).cpu().numpy().copy() for k, v in items}

    def issue(self, stream):
        L, o, s, a = _lib.lib(), self.out, self.state, self.amax
        T, N = _lib.OP_T, _lib.OP_N
        st = ctypes.c_void_p(stream)
        p = lambda x: x.data_ptr()
        keep = []

        def tn(*args, **kw):
            x = _lib.tensor(*args, **kw)
            keep.append(x)
            return ctypes.byref(x)

        def ok(status, what):
            assert status == _lib.OK, (what, _lib.status_string(status), _lib.last_error())
        # FP8 codes with the data's own amax: X per tensor (E4M3), W per row (E5M2)
        ok(L.e5ma_quantize(tn(p(self.X), F32), tn(p(o["Xq"]), E4), 512, K, 448.0, p(o["sx"]), p(o["ax"]), st),
           "quantize per tensor")
        ok(L.e5ma_quantize(tn(p(self.W), F32), tn(p(o["Wq"]), E5, scaling=_lib.SCALING_OUTER), 1024, K, 57344.0,
                           p(o["sw"]), p(o["aw"]), st), "quantize per row")
        A = lambda: tn(p(o["Wq"]), E5, p(o["sw"]), scaling=_lib.SCALING_OUTER)
        B = lambda: tn(p(o["Xq"]), E4, p(o["sx"]))
        # FP8 matrix cores (k = 8192): W . X^T with per-row scales of W, BF16 D with a BF16 bias
        ok(L.e5ma_gemm(T, N, 1024, 512, K, 1.0, A(), K, B(), K, 0.0, None, 0, tn(p(o["D1"]), B16), 1024,
                       tn(p(self.bias16), B16), st), "gemm bf16 out")
        # the same product to E5M2 with scale and amax
        ok(L.e5ma_gemm(T, N, 1024, 512, K, 1.0, A(), K, B(), K, 0.0, None, 0,
                       tn(p(o["D2"]), E5, None, p(self.q2), p(a["a2"])), 1024, None, st), "gemm e5m2 out")
        # BF16 matrix cores (k = 1024 < 8192), accumulating into an FP32 D (beta = 1, C = NULL)
        ok(L.e5ma_gemm(T, N, 1024, 512, 1024, 0.5, A(), K, B(), K, 1.0, None, 0, tn(p(s["D3"]), F32), 1024, None,
                       st), "gemm accumulate")
        # 4 tiles: split-K on a workspace and on the library's scratch
        ok(L.e5ma_gemm_ex(T, N, 512, 512, K, 1.0, A(), K, B(), K, 0.0, None, 0, tn(p(o["D4"]), F32), 512,
                          tn(p(self.bias32), F32), p(self.ws), self.ws_bytes, st), "gemm_ex")
        ok(L.e5ma_gemm_noalloc(T, N, 512, 512, K, 1.0, A(), K, B(), K, 0.0, None, 0, tn(p(o["D5"]), F32), 512,
                               tn(p(self.bias32), F32), st), "gemm_noalloc")
        # GEMV n = 1 and n = 8 with a BF16 x
        ok(L.e5ma_gemm(T, N, 1024, 1, K, 1.0, A(), K, tn(p(self.x1), B16), K, 0.0, None, 0, tn(p(o["D6"]), F32),
                       1024, None, st), "gemv n=1")
        ok(L.e5ma_gemm(T, N, 1024, 8, K, 1.0, A(), K, tn(p(self.x8), B16), K, 0.0, None, 0, tn(p(o["D7"]), B16),
                       1024, None, st), "gemv n=8")
        # cast FP32 -> E5M2 with scale and amax
        ok(L.e5ma_cast(tn(p(self.Xc), F32), tn(p(o["Cc"]), E5, None, p(self.qc), p(a["ac"])), 1 << 20, st), "cast")
        # AdamW on BF16 parameters with FP32 state and an E4M3 copy of the new weights
        cfg = _lib.AdamConfig(1e-3, 0.9, 0.999, 1e-8, 0.01, 5, 1, 1, 1.0)
        ok(L.e5ma_adam(ctypes.byref(cfg), (1 << 20) + 3, tn(p(s["P"]), B16), tn(p(self.G), F32),
                       tn(p(s["M"]), F32), tn(p(s["V"]), F32), tn(p(o["Q"]), E4, None, p(self.qa), p(a["aa"])), st),
           "adam")


def test_graph_replays_match_eager(dev):
    rng = np.random.default_rng(0x6A4F)
    c = Calls(dev, rng)
    # eager: also initializes the library on this device before any capture
    c.reset()
    torch.cuda.synchronize(dev)
    c.issue(torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize(dev)
    eager = c.snapshot()
    for k, v in eager.items():
        if k in c.out:
            assert not np.all(v == 0xA5), f"{k} was not written"
    # two eager results against the oracle: per-tensor quantize of X, GEMV n = 1
    codes, sinv, amax = oracle.quantize(F32, E4, c.X.cpu().numpy(), 512, K, 448.0)
    assert np.array_equal(eager["Xq"], codes)
    assert np.array_equal(eager["sx"].view(np.float32), sinv) and np.array_equal(eager["ax"].view(np.float32), amax)
    Wq = eager["Wq"]
    sw = eager["sw"].view(np.float32)
    case = gu.GemmCase(rng, 1, 0, 1024, 1, K, E5, B16, sa=sw, A=Wq, B=c.x1.cpu().numpy().view(np.uint16), pad=0,
                       ldd=1024)
    bad, first = case.check(eager["D6"].view(np.float32))
    assert bad == 0, first

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.graph(graph, stream=side):
        c.issue(torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize(dev)
    y = torch.randn(1024, 1024, device=dev)
    for replay in range(4):
        c.reset()
        graph.replay()
        y = torch.tanh(y @ y.T / 1024)  # the program's own eager work between replays
        torch.cuda.synchronize(dev)
        got = c.snapshot()
        for k in eager:
            assert np.array_equal(got[k], eager[k]), \
                f"replay {replay}: {k} differs at {np.count_nonzero(got[k] != eager[k])} bytes"
    del graph
