"""The Python layer (matmul / linear / cast / adam_step / AdamW / Float8Tensor / quantize_linear_) on the
GPU.  Results are held to a float64 product with the bound
|y - ref| <= half an output ulp * |ref| + k * 2^-23 * sum|a*b| (the contract's FP32 accumulation error),
codecs are compared with torch's own conversions, and the optimizer with torch.optim.AdamW.  Mirrors the
coverage of the reference's binds/python/tests/test_e5m2effma.py:42-336."""
import pytest
import torch
import torch.nn.functional as Fn

import e5m2effma_amd as fx

pytestmark = pytest.mark.gpu
DEV = "cuda"
F8, F4 = torch.float8_e5m2, torch.float8_e4m3fn
TOP = {F8: 57344.0, F4: 448.0}
HALF_ULP = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -24, F8: 2.0 ** -3,
            F4: 2.0 ** -4}


def rand(shape, dtype, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(DEV).to(dtype)


def within_bound(y, ref, mag, k, out_dtype):
    err = (y.double() - ref).abs()
    bound = HALF_ULP[out_dtype] * ref.abs() + k * 2.0 ** -23 * mag + 1e-30
    excess = (err - bound * 1.0001).max()
    assert float(excess) <= 0, f"bound exceeded by {float(excess)}"


def product(a, b, sa=1.0, sb=1.0, bias=None):
    A, B = a.double() * sa, b.double() * sb
    r = A @ B
    if bias is not None:
        r = r + bias.double()
    return r, A.abs() @ B.abs()


OPS = [F8, F4, torch.bfloat16, torch.float32]


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("b_layout", ["row", "col"])
@pytest.mark.parametrize("tb", OPS)
@pytest.mark.parametrize("ta", OPS)
def test_matmul(ta, tb, b_layout, out_dtype):
    M, K, N = 70, 96, 50
    a = rand((M, K), ta, seed=1)
    b = rand((K, N), tb, seed=2) if b_layout == "row" else rand((N, K), tb, seed=2).t()
    y = fx.matmul(a, b, out_dtype=out_dtype)
    assert y.shape == (M, N) and y.dtype == out_dtype
    within_bound(y, *product(a, b), K, out_dtype)


@pytest.mark.parametrize("tw", [F8, F4])
@pytest.mark.parametrize("tx", OPS)
@pytest.mark.parametrize("rows", [1, 3, 8, 9, 64])
def test_linear_fp8_weight(rows, tx, tw):  # rows <= 8: the GEMV kernel
    N, K = 300, 512
    w, x = rand((N, K), tw, seed=3), rand((rows, K), tx, seed=4)
    bias = rand((N,), torch.bfloat16, seed=5)
    y = fx.linear(x, w, bias, scale_w=torch.tensor([0.25], device=DEV))
    within_bound(y, *product(x, w.t(), sb=0.25, bias=bias), K, torch.bfloat16)


def test_linear_batched_shape():
    assert fx.linear(rand((2, 3, 64), torch.bfloat16), rand((40, 64), F8, seed=1)).shape == (2, 3, 40)


def test_accumulate_into_fp32_out():
    M, K, N = 33, 64, 47
    a, b = rand((M, K), torch.bfloat16, seed=1), rand((K, N), torch.bfloat16, seed=2)
    out = rand((M, N), torch.float32, seed=3)
    start = out.clone()
    fx.matmul(a, b, out=out, beta=1.0)
    ref, mag = product(a, b)
    within_bound(out, ref + start.double(), mag + start.double().abs(), K, torch.float32)


@pytest.mark.parametrize("out", [F8, F4])
def test_fp8_output_scale_amax(out):
    M, K, N = 16, 64, 32
    a, b = rand((M, K), F8, seed=1), rand((K, N), F4, seed=2)
    scale, amax = torch.tensor([4.0], device=DEV), torch.zeros(1, device=DEV)
    y = fx.matmul(a, b, out_dtype=out, scale_out=scale, amax_out=amax)
    ref, _ = product(a, b)
    assert y.dtype == out
    assert float(amax) == pytest.approx(float(ref.abs().max()), rel=2 ** -20)
    expect = (ref * 4.0).clamp(-TOP[out], TOP[out]).float().to(out)
    assert torch.equal(y.view(torch.uint8), expect.view(torch.uint8))


@pytest.mark.parametrize("dtype", [F8, F4, torch.bfloat16, torch.float16])
def test_cast_matches_torch(dtype):
    x = rand((1000, 37), torch.float32, scale=50.0).clamp(-448, 448)
    assert torch.equal(fx.cast(x, dtype).view(torch.uint8), x.to(dtype).view(torch.uint8))


@pytest.mark.parametrize("dtype", [F8, F4])
def test_cast_scale_roundtrip(dtype):
    x = rand((4096,), torch.float32)
    amax, scale = torch.zeros(1, device=DEV), torch.tensor([64.0], device=DEV)
    q = fx.cast(x, dtype, scale=scale, amax=amax)
    assert float(amax) == float(x.abs().max())
    back = fx.cast(q, torch.float32, scale_inv=torch.tensor([1 / 64.0], device=DEV))
    assert torch.equal(back, (x * 64).to(dtype).float() / 64)


def test_cast_e5m2_inf_nan_and_kat():
    codes = torch.arange(256, device=DEV, dtype=torch.uint8).view(F8)
    y = fx.cast(codes, torch.float32)
    assert torch.equal(y.isinf(), codes.float().isinf()) and torch.equal(y.isnan(), codes.float().isnan())
    amax = torch.zeros(1, device=DEV)
    q = fx.cast(torch.tensor([1.0, float("inf"), -1e6, 3.0], device=DEV), F8, amax=amax)
    assert q.view(torch.uint8).tolist() == [0x3C, 0x7B, 0xFB, 0x42] and float(amax) == float("inf")


@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("pdtype", [torch.float32, torch.bfloat16])
def test_adamw_against_torch(pdtype, state_dtype):
    torch.manual_seed(0)
    ref = torch.nn.Parameter(torch.randn(1000, device=DEV))
    mine = torch.nn.Parameter(ref.detach().clone().to(pdtype))
    opt_ref = torch.optim.AdamW([ref], lr=1e-2, weight_decay=0.1, foreach=False)
    opt = fx.AdamW([mine], lr=1e-2, weight_decay=0.1, state_dtype=state_dtype)
    for _ in range(5):
        g = torch.randn(1000, device=DEV)
        ref.grad, mine.grad = g.clone(), g.to(pdtype)
        opt_ref.step()
        opt.step()
    tol = 1e-6 if pdtype == torch.float32 and state_dtype == torch.float32 else 2e-2
    torch.testing.assert_close(mine.detach().float(), ref.detach(), rtol=tol, atol=tol)
    assert opt.state[mine]["exp_avg"].dtype == state_dtype and opt.state[mine]["step"] == 5


@pytest.mark.parametrize("qt", [F8, F4])
def test_adam_step_fp8_copy(qt):
    p = rand((256,), torch.float32)
    g, m, v = rand((256,), torch.bfloat16, seed=1), torch.zeros(256, device=DEV), torch.zeros(256, device=DEV)
    q, amax = torch.empty(256, device=DEV, dtype=qt), torch.zeros(1, device=DEV)
    fx.adam_step(p, g, m, v, lr=1e-3, step=1, param_fp8=q, fp8_scale=torch.tensor([8.0], device=DEV), fp8_amax=amax)
    assert torch.equal(q.view(torch.uint8), (p * 8).to(qt).view(torch.uint8))
    assert float(amax) == float(p.abs().max())


@pytest.mark.parametrize("which", ["a", "b", "both"])
def test_matmul_rowwise_scales(which):
    M, K, N = 70, 96, 50
    a, b = rand((M, K), F8, seed=1), rand((N, K), F4, seed=2).t()
    sa = torch.rand(M, device=DEV) + 0.5 if which in ("a", "both") else torch.tensor([0.75], device=DEV)
    sb = torch.rand(N, device=DEV) + 0.5 if which in ("b", "both") else torch.tensor([1.5], device=DEV)
    for out_dtype in (torch.bfloat16, torch.float32):
        y = fx.matmul(a, b, scale_a=sa, scale_b=sb, out_dtype=out_dtype)
        sa2 = sa.double().reshape(-1, 1) if sa.numel() > 1 else sa.double()
        sb2 = sb.double().reshape(1, -1) if sb.numel() > 1 else sb.double()
        within_bound(y, *product(a, b, sa2, sb2), K, out_dtype)


@pytest.mark.parametrize("rows", [1, 8, 64])
def test_linear_per_channel_weight_scale(rows):
    N, K = 300, 512
    w, x = rand((N, K), F8, seed=3), rand((rows, K), torch.bfloat16, seed=4)
    sw = torch.rand(N, device=DEV) + 0.5
    y = fx.linear(x, w, scale_w=sw)
    within_bound(y, *product(x, w.t(), sb=sw.double().reshape(1, -1)), K, torch.bfloat16)


# ---- Float8Tensor ---------------------------------------------------------------------------------
@pytest.mark.parametrize("rows", [1, 8, 64])
@pytest.mark.parametrize("per_row", [False, True])
@pytest.mark.parametrize("fp8", [F8, F4])
def test_float8tensor_linear(fp8, per_row, rows):
    w, x = rand((300, 512), torch.bfloat16, seed=3), rand((rows, 512), torch.bfloat16, seed=4)
    w8 = fx.Float8Tensor.from_float(w, fp8=fp8, per_row=per_row)
    assert isinstance(w8, fx.Float8Tensor) and w8.dtype == torch.bfloat16 and w8.shape == w.shape
    assert w8._data.dtype == fp8
    bias = rand((300,), torch.bfloat16, seed=5)
    y = Fn.linear(x, w8, bias)
    assert y.dtype == torch.bfloat16 and not isinstance(y, fx.Float8Tensor)
    s = w8._scale_inv if per_row else w8._scale_inv.reshape(())
    assert torch.equal(y, fx.linear(x, w8._data, scale_w=s, bias=bias))  # the same kernel call
    assert torch.equal(x @ w8.t() + 0, fx.linear(x, w8._data, scale_w=s))
    wd = w8.dequantize(torch.float64)
    within_bound(y, x.double() @ wd.t() + bias.double(), x.double().abs() @ wd.abs().t(), 512, torch.bfloat16)


def test_float8tensor_both_operands():
    a8 = fx.Float8Tensor.from_float(rand((70, 96), torch.float32, seed=1), per_row=True, dtype=torch.float32)
    b8 = fx.Float8Tensor.from_float(rand((50, 96), torch.float32, seed=2), per_row=True, dtype=torch.float32)
    y = a8 @ b8.t()  # per-row scales of both operands are outer: one FP8 x FP8 GEMM
    assert y.dtype == torch.float32
    assert torch.equal(y, fx.matmul(a8._data, b8._data.t(), scale_a=a8._scale_inv, scale_b=b8._scale_inv,
                                    out_dtype=torch.float32))
    ad, bd = a8.dequantize(torch.float64), b8.dequantize(torch.float64)
    within_bound(y, ad @ bd.t(), ad.abs() @ bd.abs().t(), 96, torch.float32)
    # a scale along K (a8 as the right operand without transpose) can only be applied by dequantizing
    z = b8.t().t() @ a8.t()
    assert torch.allclose(z, b8.float() @ a8.float().t(), rtol=1e-5, atol=1e-4)
    w = a8.t() @ a8  # both scales run along K: dequantized product
    assert torch.allclose(w, a8.float().t() @ a8.float(), rtol=1e-5, atol=1e-4)


def test_quantize_linear_module():
    torch.manual_seed(0)
    m = torch.nn.Sequential(torch.nn.Linear(512, 256), torch.nn.GELU(), torch.nn.Linear(256, 64),
                            torch.nn.Linear(64, 8, bias=False), torch.nn.Linear(8, 8)).to(DEV, torch.bfloat16)
    x = rand((4, 7, 512), torch.bfloat16, seed=6)
    with torch.no_grad():
        ref = m(x).float()
        fx.quantize_linear_(m)
        y = m(x).float()
    assert [isinstance(l.weight, fx.Float8Tensor) for l in m if isinstance(l, torch.nn.Linear)] == \
        [True, True, True, False]  # in_features 8 is not a multiple of 16: kept
    assert float((y - ref).norm() / ref.norm()) < 0.1


def test_float8tensor_from_float_per_row_needs_2d():
    with pytest.raises(ValueError, match="per_row"):
        fx.Float8Tensor.from_float(torch.ones(2, 3, 16, device=DEV), per_row=True)


# ---- rejection of bad input -----------------------------------------------------------------------
def test_rejects_bad_dtype_and_shapes():
    with pytest.raises(TypeError):
        fx.matmul(torch.zeros(16, 16, device=DEV, dtype=torch.float64), rand((16, 16), F8))
    with pytest.raises(TypeError):
        fx.matmul(rand((16, 16), torch.float16), rand((16, 16), F8))
    with pytest.raises(ValueError, match="shapes"):
        fx.matmul(rand((8, 32), F8), rand((16, 8), F8))
    with pytest.raises(ValueError, match="shape"):
        fx.linear(rand((4, 32), torch.bfloat16), rand((8, 48), F8))
    with pytest.raises(ValueError, match="multiple of 16"):
        fx.matmul(rand((8, 24), F8), rand((24, 8), F8))


@pytest.mark.parametrize("view", ["offset", "strided", "row_major_n_not_16"])
def test_awkward_layouts_are_repacked(view):
    base = rand((40, 130), F8, seed=7)
    a = {"offset": base[:, 1:129], "strided": base[:, ::2][:, :64], "row_major_n_not_16": base[:, :128]}[view]
    b = rand((a.shape[1], 50), torch.bfloat16, seed=8)
    y = fx.matmul(a, b)
    assert torch.equal(y, fx.matmul(a.contiguous(), b.t().contiguous().t()))
    within_bound(y, *product(a, b), a.shape[1], torch.bfloat16)


def test_rejects_misused_scales_and_out():
    with pytest.raises(ValueError, match="scale_a"):
        fx.matmul(rand((8, 16), torch.bfloat16), rand((16, 8), F8), scale_a=torch.ones(1, device=DEV))
    with pytest.raises(TypeError, match="float32"):
        fx.matmul(rand((8, 16), F8), rand((16, 8), F8), scale_a=torch.ones(1, device=DEV, dtype=torch.float64))
    with pytest.raises(ValueError, match="one element"):
        fx.matmul(rand((8, 16), F8), rand((16, 8), F8), scale_a=torch.ones(2, device=DEV))
    a, b = rand((8, 16), F8), rand((16, 8), F8)
    with pytest.raises(ValueError, match="out must be given"):
        fx.matmul(a, b, beta=1.0)
    with pytest.raises(ValueError, match="shape"):
        fx.matmul(a, b, out=torch.empty(8, 9, device=DEV, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="row-contiguous"):
        fx.matmul(a, b, out=torch.empty(8, 8, device=DEV, dtype=torch.bfloat16).t())
    x = rand((16, 16), torch.float32)
    with pytest.raises(ValueError, match="share memory"):
        fx.matmul(x, rand((16, 16), torch.float32, seed=1), out=x)


def test_rejects_adam_problems():
    p, g = rand((10,), torch.float32), rand((10,), torch.float32)
    m, v = torch.zeros(10, device=DEV), torch.zeros(10, device=DEV)
    with pytest.raises(ValueError, match="step"):
        fx.adam_step(p, g, m, v, lr=1e-3, step=0)
    with pytest.raises(ValueError, match="elements"):
        fx.adam_step(p, g[:5], m, v, lr=1e-3, step=1)
    with pytest.raises(TypeError, match="exp_avg_sq"):
        fx.adam_step(p, g, m, v.bfloat16(), lr=1e-3, step=1)
    with pytest.raises(ValueError, match="share memory"):
        fx.adam_step(p, g, m, m, lr=1e-3, step=1)
    with pytest.raises(ValueError, match="betas"):
        fx.adam_step(p, g, m, v, lr=1e-3, betas=(0.9, 1.0), step=1)
