"""The torch layer (e5m2effma_amd: matmul, linear, cast, adam_step, AdamW, Float8Tensor, quantize_linear_)
on the GPU, checked against the CPU oracle: GEMM results against the accumulation bound, casts, Adam steps
and quantization bit for bit.  Row-major products are checked as the column-major GEMM the layer issues
(out^T = b^T a^T, reference binds/python/csrc/e5m2effma_torch.cpp:179-197)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import e5m2effma_amd as fx
import gpu_util as gu
import oracle

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
CODE = {torch.float8_e5m2: oracle.E5M2, torch.float8_e4m3fn: oracle.E4M3, torch.bfloat16: oracle.BF16,
        torch.float16: oracle.FP16, torch.float32: oracle.FP32}
NPV = {torch.float8_e5m2: np.uint8, torch.float8_e4m3fn: np.uint8, torch.bfloat16: np.uint16,
       torch.float16: np.uint16, torch.float32: np.float32}
RAW = {np.uint8: torch.uint8, np.uint16: torch.int16, np.float32: torch.float32}


def host(t):
    """A tensor's elements as the oracle's numpy codes (row-major, contiguous)."""
    t = t.detach().contiguous()
    raw = t.view(RAW[NPV[t.dtype]]) if t.dtype != torch.float32 else t
    return raw.cpu().numpy().view(NPV[t.dtype]).ravel().copy()


def device(codes, dtype, shape):
    t = torch.from_numpy(np.ascontiguousarray(codes).view(np.uint8 if NPV[dtype] == np.uint8 else NPV[dtype]))
    if dtype == torch.float32:
        return t.reshape(shape).to(DEV)
    return t.view(RAW[NPV[dtype]]).reshape(shape).to(DEV).view(dtype)


def operand(rng, dtype, shape, sigma=2.0):
    n = int(np.prod(shape))
    if dtype in (torch.float8_e5m2, torch.float8_e4m3fn):
        return device(gu.normal_fp8(rng, n, CODE[dtype], sigma), dtype, shape)
    x = (rng.standard_normal(n) * sigma).astype(np.float32)
    return device(x if dtype == torch.float32 else oracle.encode(CODE[dtype], x), dtype, shape)


def check_product(a, b, out, *, alpha=1.0, beta=0.0, out0=None, bias=None, scale_a=None, scale_b=None,
                  scale_out=None, amax=None):
    """out (row-major [M, N]) against the oracle bound for alpha * (sa * sb) * (a @ b) + bias + beta * out0."""
    M, K = a.shape
    N = b.shape[1]
    sa = None if scale_a is None else host(scale_a.float())
    sb = None if scale_b is None else host(scale_b.float())
    D0 = host(out0) if out0 is not None else np.zeros(M * N, NPV[out.dtype])
    g = oracle.Gemm(1, 0, N, M, K, alpha, CODE[b.dtype], host(b.t()), K, CODE[a.dtype], host(a), K,
                    sa=sb, sa_vec=sb is not None and sb.size > 1, sb=sa, sb_vec=sa is not None and sa.size > 1,
                    beta=beta, ddt=CODE[out.dtype], D=D0.copy(), ldd=N,
                    qscale=1.0 if scale_out is None else float(scale_out.item()),
                    biasdt=CODE[bias.dtype] if bias is not None else oracle.FP32,
                    bias=None if bias is None else host(bias), ocp_operands=True)
    iis, jjs = [v.ravel() for v in np.meshgrid(np.arange(N), np.arange(M), indexing="ij")]
    bad, first, alo, ahi = g.check(host(out), D0 if beta != 0.0 else None, iis, jjs)
    assert bad == 0, (bad, first)
    if amax is not None:
        got = float(amax.item())
        assert alo <= got <= ahi or got == alo == ahi, (got, alo, ahi)


@pytest.mark.parametrize("adt,bdt,odt", [(torch.float8_e5m2, torch.float8_e4m3fn, torch.bfloat16),
                                         (torch.float8_e4m3fn, torch.float8_e5m2, torch.float32),
                                         (torch.float8_e5m2, torch.bfloat16, torch.float16),
                                         (torch.bfloat16, torch.float8_e4m3fn, torch.bfloat16)])
@pytest.mark.parametrize("b_t", [False, True])
def test_matmul_pairings_and_b_layouts(adt, bdt, odt, b_t):
    rng = np.random.default_rng(100 * CODE[adt] + 10 * CODE[bdt] + int(b_t))
    M, K, N = 72, 96, 40
    a = operand(rng, adt, (M, K))
    b = operand(rng, bdt, (N, K)).t() if b_t else operand(rng, bdt, (K, N))
    sa = torch.tensor([0.75], device=DEV) if adt in (torch.float8_e5m2, torch.float8_e4m3fn) else None
    sb = torch.tensor([1.5], device=DEV) if bdt in (torch.float8_e5m2, torch.float8_e4m3fn) else None
    out = fx.matmul(a, b, out_dtype=odt, scale_a=sa, scale_b=sb, alpha=0.5)
    assert out.shape == (M, N) and out.dtype == odt
    check_product(a, b, out, alpha=0.5, scale_a=sa, scale_b=sb)


def test_matmul_bias_accumulate_and_fp8_output():
    rng = np.random.default_rng(5)
    M, K, N = 64, 128, 48
    a, b = operand(rng, torch.float8_e4m3fn, (M, K)), operand(rng, torch.float8_e5m2, (K, N))
    bias = operand(rng, torch.bfloat16, (N,))
    acc = operand(rng, torch.float32, (M, N), sigma=4.0)
    acc0 = acc.clone()
    fx.matmul(a, b, out=acc, beta=1.0, bias=bias)
    check_product(a, b, acc, beta=1.0, out0=acc0, bias=bias)
    so, am = torch.tensor([0.125], device=DEV), torch.zeros(1, device=DEV)
    o8 = fx.matmul(a, b, out_dtype=torch.float8_e5m2, scale_out=so, amax_out=am)
    check_product(a, b, o8, scale_out=so, amax=am)


@pytest.mark.parametrize("which", ["a", "b", "both"])
def test_matmul_row_and_column_scales(which):
    rng = np.random.default_rng(len(which))
    M, K, N = 80, 64, 56
    a, b = operand(rng, torch.float8_e5m2, (M, K)), operand(rng, torch.float8_e4m3fn, (K, N))
    sa = torch.from_numpy(rng.uniform(0.25, 2, M).astype(np.float32)).to(DEV) if which != "b" else None
    sb = torch.from_numpy(rng.uniform(0.25, 2, N).astype(np.float32)).to(DEV) if which != "a" else None
    out = fx.matmul(a, b, scale_a=sa, scale_b=sb)
    check_product(a, b, out, scale_a=sa, scale_b=sb)


@pytest.mark.parametrize("rows", [1, 5, 8, 33])
def test_linear_with_per_channel_weight_scale(rows):
    """rows <= 8 run the GEMV kernel (x row-major, W FP8 K-contiguous), more rows the tiled GEMM."""
    rng = np.random.default_rng(rows)
    K, Nout = 256, 96
    x = operand(rng, torch.bfloat16, (rows, K), sigma=1.0)
    w = operand(rng, torch.float8_e4m3fn, (Nout, K))
    sw = torch.from_numpy(rng.uniform(0.01, 0.05, Nout).astype(np.float32)).to(DEV)
    bias = operand(rng, torch.float32, (Nout,))
    y = fx.linear(x, w, bias, scale_w=sw)
    assert y.shape == (rows, Nout)
    check_product(x, w.t(), y, bias=bias, scale_b=sw)


def test_linear_keeps_leading_dims():
    rng = np.random.default_rng(9)
    x = operand(rng, torch.bfloat16, (2, 3, 64))
    w = operand(rng, torch.float8_e5m2, (32, 64))
    y = fx.linear(x, w)
    assert y.shape == (2, 3, 32)
    check_product(x.reshape(6, 64), w.t(), y.reshape(6, 32))


def test_large_product_splits_k_with_a_torch_workspace():
    """A 4-tile output at k = 8192 runs e5ma_gemm_ex with a split-K workspace from torch's allocator."""
    rng = np.random.default_rng(11)
    M = N = 512
    K = 8192
    a, b = operand(rng, torch.float8_e5m2, (M, K), 4.0), operand(rng, torch.float8_e4m3fn, (K, N), 4.0)
    # row-major a, b issue e5ma_gemm_ex(N, N, N, M, K) with A := b (lda N), B := a (ldb K)
    assert fx._lib.workspace_size(0, 0, N, M, K, oracle.E4M3, N, oracle.E5M2, K) > 0
    out = fx.matmul(a, b, out_dtype=torch.float32)
    check_product(a, b, out)


@pytest.mark.parametrize("src,dst", [(torch.float32, torch.float8_e5m2), (torch.bfloat16, torch.float8_e4m3fn),
                                     (torch.float8_e5m2, torch.float32), (torch.float8_e4m3fn, torch.bfloat16)])
def test_cast_is_the_oracle_cast(src, dst):
    rng = np.random.default_rng(3)
    x = operand(rng, src, (1000, 3), sigma=300.0)
    si = torch.tensor([0.5], device=DEV) if src in (torch.float8_e5m2, torch.float8_e4m3fn) else None
    sc = torch.tensor([0.25], device=DEV) if dst in (torch.float8_e5m2, torch.float8_e4m3fn) else None
    am = torch.zeros(1, device=DEV)
    y = fx.cast(x, dst, scale_inv=si, scale=sc, amax=am)
    want, want_amax = oracle.cast(CODE[src], CODE[dst], host(x), x.numel(), 1.0 if si is None else 0.5,
                                  1.0 if sc is None else 0.25)
    assert np.array_equal(host(y), want) and np.float32(am.item()) == np.float32(want_amax)


@pytest.mark.parametrize("pdt,sdt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                     (torch.float32, torch.bfloat16)])
def test_adamw_optimizer_matches_the_oracle(pdt, sdt):
    """Three steps of fx.AdamW over two parameters (one with a grad scale group option), bit for bit
    against the oracle's element order."""
    rng = np.random.default_rng(17)
    shapes = [(33, 17), (1000,)]
    params = [torch.nn.Parameter(operand(rng, pdt, s, 0.5)) for s in shapes]
    opt = fx.AdamW(params, lr=1e-3, weight_decay=0.05, state_dtype=sdt, grad_scale=0.5)
    ref = [dict(p=host(p), m=np.zeros(p.numel(), NPV[sdt]), v=np.zeros(p.numel(), NPV[sdt])) for p in params]
    for step in range(1, 4):
        for p, r in zip(params, ref):
            g = operand(rng, pdt, p.shape, 1e-2)  # torch ties .grad's dtype to the parameter's
            p.grad = g
            r["g"] = host(g)
        opt.step()
        cfg = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.05, step=step, adamw=1,
                   bias_correction=1, grad_scale=0.5)
        for p, r in zip(params, ref):
            oracle.adam(cfg, CODE[pdt], r["p"], CODE[pdt], r["g"], CODE[sdt], r["m"], r["v"], threads=4)
            st = opt.state[p]
            assert st["step"] == step
            assert np.array_equal(host(p.data), r["p"]), f"param after step {step}"
            assert np.array_equal(host(st["exp_avg"]), r["m"]) and np.array_equal(host(st["exp_avg_sq"]), r["v"])


def test_adamw_fp8_copy_with_delayed_scaling():
    """fp8_copy: each step's copy is the updated weights quantized with the previous step's amax."""
    rng = np.random.default_rng(23)
    p = torch.nn.Parameter(operand(rng, torch.float32, (4096,), 0.02))
    opt = fx.AdamW([p], lr=1e-3, fp8_copy=torch.float8_e4m3fn)
    amax_prev = float(p.detach().abs().max())
    for step in range(1, 4):
        p.grad = operand(rng, torch.float32, (4096,), 1e-3)
        opt.step()
        st = opt.state[p]
        scale = np.float32(st["fp8_scale"].item())  # torch's 448 / amax: reciprocal() * 448 on the device
        assert scale == pytest.approx(448.0 / max(amax_prev, 1e-12), rel=2e-7)
        w = host(p.data)
        assert np.array_equal(host(st["param_fp8"]), oracle.encode(oracle.E4M3, w, float(scale)))
        amax_prev = float(np.abs(w).max())
        assert np.float32(st["fp8_amax"].item()) == np.float32(amax_prev)
        assert float(st["fp8_scale_inv"].item()) == pytest.approx(1.0 / float(scale), rel=2e-7)


@pytest.mark.parametrize("fp8,per_row", [(torch.float8_e4m3fn, True), (torch.float8_e5m2, False)])
def test_float8tensor_from_float_and_products(fp8, per_row):
    rng = np.random.default_rng(int(per_row) + 7)
    w = torch.from_numpy((rng.standard_normal((96, 128)) * 0.05).astype(np.float32)).to(DEV)
    q = fx.Float8Tensor.from_float(w, fp8=fp8, per_row=per_row, dtype=torch.bfloat16)
    codes, sinv, _ = oracle.quantize(oracle.FP32, CODE[fp8], host(w), 96, 128,
                                     57344.0 if fp8 == torch.float8_e5m2 else 448.0, per_row=per_row)
    assert np.array_equal(host(q.codes), codes) and np.array_equal(host(q.scale_inv), sinv)
    x = operand(rng, torch.bfloat16, (40, 128), 1.0)
    bias = operand(rng, torch.bfloat16, (96,), 1.0)
    for y in (F.linear(x, q, bias), torch.addmm(bias, x, q.t()), x @ q.t() + 0 * bias):
        assert type(y) is torch.Tensor and y.dtype == torch.bfloat16 and y.shape == (40, 96)
    y = F.linear(x, q, bias)
    check_product(x, q.codes.t(), y, bias=bias, scale_b=q.scale_inv)
    y2 = torch.addmm(bias, x, q.t(), alpha=0.5)
    check_product(x, q.codes.t(), y2, alpha=0.5, bias=bias, scale_b=q.scale_inv)


def test_float8tensor_both_operands_fp8():
    rng = np.random.default_rng(29)
    a32 = torch.from_numpy((rng.standard_normal((64, 96)) * 3).astype(np.float32)).to(DEV)
    b32 = torch.from_numpy((rng.standard_normal((80, 96)) * 0.1).astype(np.float32)).to(DEV)
    qa = fx.Float8Tensor.from_float(a32, fp8=torch.float8_e5m2, per_row=True, dtype=torch.float32)
    qb = fx.Float8Tensor.from_float(b32, fp8=torch.float8_e4m3fn, per_row=True, dtype=torch.float32)
    y = qa @ qb.t()
    assert y.dtype == torch.float32
    check_product(qa.codes, qb.codes.t(), y, scale_a=qa.scale_inv, scale_b=qb.scale_inv)


def test_quantize_linear_module():
    rng = np.random.default_rng(31)
    torch.manual_seed(0)
    model = torch.nn.Sequential(torch.nn.Linear(64, 48), torch.nn.ReLU(), torch.nn.Linear(48, 24),
                                torch.nn.Linear(24, 8)).to(DEV).to(torch.bfloat16)
    fx.quantize_linear_(model)
    l0, l2, l3 = model[0], model[2], model[3]
    assert isinstance(l0.weight, fx.Float8Tensor) and isinstance(l2.weight, fx.Float8Tensor)
    assert not isinstance(l3.weight, fx.Float8Tensor)  # in_features 24 is not a multiple of 16
    assert l0.weight.codes.dtype == torch.float8_e4m3fn and l0.weight.scale_dim == 0
    x = operand(rng, torch.bfloat16, (16, 64), 1.0)
    h = model[0](x)
    check_product(x, l0.weight.codes.t(), h, bias=l0.bias, scale_b=l0.weight.scale_inv)
    assert model(x).shape == (16, 8)


@pytest.mark.parametrize("call,exc,text", [
    (lambda: fx.matmul(torch.zeros(16, 16, device=DEV, dtype=torch.float16), torch.zeros(16, 16, device=DEV)),
     TypeError, "float16"),
    (lambda: fx.matmul(torch.zeros(16, 24, device=DEV), torch.zeros(24, 16, device=DEV)), ValueError, "multiple of 16"),
    (lambda: fx.matmul(torch.zeros(16, 16, device=DEV), torch.zeros(32, 16, device=DEV)), ValueError, "shapes"),
    (lambda: fx.matmul(torch.zeros(16, 16, device=DEV), torch.zeros(16, 16, device=DEV), beta=1.0),
     ValueError, "out must be given"),
    (lambda: fx.adam_step(*(torch.zeros(4, device=DEV) for _ in range(4)), lr=1e-3, step=0), ValueError, "step"),
    (lambda: fx.cast(torch.zeros(4, device=DEV), torch.int8), TypeError, "dtype"),
])
def test_errors_map_to_python_exceptions(call, exc, text):
    with pytest.raises(exc, match=text):
        call()
