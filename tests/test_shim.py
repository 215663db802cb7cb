"""The Python layer's host-side behaviour (no GPU): Float8Tensor's stored form, the operations it keeps in
FP8 and the ones it dequantizes, AdamW's argument checks, the dtype alias and the rejection of CPU
tensors (the reference pins the same behaviour in binds/python/tests/test_e5m2effma.py:254-336)."""
import pytest
import torch

import e5m2effma_amd as fx

F8, F4 = torch.float8_e5m2, torch.float8_e4m3fn


def codes_4x16(fmt=F8):
    return torch.arange(64, dtype=torch.uint8).reshape(4, 16).view(fmt)


def test_dtype_alias_and_exports():
    assert torch.e5m2effma is torch.float8_e5m2 and fx.e5m2 is torch.float8_e5m2 and fx.e4m3 is torch.float8_e4m3fn
    for name in ("matmul", "linear", "cast", "quantize", "adam_step", "AdamW", "Float8Tensor", "quantize_linear_",
                 "torch_ops_enabled", "get_include", "__version__"):
        assert name in fx.__all__ and hasattr(fx, name)


def test_get_include_and_torch_ops():
    """get_include() names the directories of the C ABI headers and the device codecs; aten::_scaled_mm is
    never overridden (gfx950 has native FP8 in PyTorch's own kernel)."""
    import os
    inc = fx.get_include()
    assert os.path.isfile(os.path.join(inc[0], "e5m2effma.h")) and os.path.isfile(os.path.join(inc[0], "e5m2effma_ext.h"))
    assert os.path.isfile(os.path.join(inc[1], "e5ma_device.hpp"))
    assert fx.torch_ops_enabled() is False


@pytest.mark.parametrize("args,exc,text", [
    ((codes_4x16().float(), torch.ones(1)), TypeError, "float8_e5m2"),
    ((codes_4x16(), torch.ones(1, dtype=torch.float64)), TypeError, "float32"),
    ((codes_4x16(), torch.ones(16), 0), ValueError, "needs 4 factors"),
    ((codes_4x16(), torch.ones(4), 2), ValueError, "rows"),
    ((codes_4x16().reshape(64), torch.ones(64), 0), ValueError, "2-D"),
    ((codes_4x16(), torch.ones(2)), ValueError, "one element"),
    ((codes_4x16(), torch.ones(1), None, torch.float64), TypeError, "nominal dtype"),
])
def test_float8tensor_rejects(args, exc, text):
    with pytest.raises(exc, match=text):
        fx.Float8Tensor(*args)


def test_from_float_needs_a_rocm_tensor_and_fp8_format():
    with pytest.raises(ValueError, match="ROCm"):
        fx.Float8Tensor.from_float(torch.ones(4, 16))
    with pytest.raises(TypeError, match="fp8"):
        fx.Float8Tensor.from_float(torch.ones(4, 16), fp8=torch.bfloat16)


def test_stored_form_and_values():
    s = torch.tensor([0.5, 1.0, 2.0, 4.0])
    x = fx.Float8Tensor(codes_4x16(), s, 0, torch.float32)
    assert x.shape == (4, 16) and x.dtype == torch.float32 and x.codes.dtype == F8 and x.scale_dim == 0
    assert x._data is x.codes and x._scale_dim == 0 and torch.equal(x._scale_inv, s)  # reference names
    want = codes_4x16().float() * s[:, None]
    assert torch.equal(x.dequantize(), want) and torch.equal(x.float(), want)
    assert x.to(torch.bfloat16).dtype == torch.bfloat16 and type(x.to(torch.bfloat16)) is torch.Tensor
    assert "per row" in repr(x) and "float8_e5m2" in repr(x)


def test_per_tensor_known_values():
    c = torch.tensor([0x3C, 0xBC, 0x40, 0x00], dtype=torch.uint8).view(F8).reshape(2, 2)  # 1, -1, 2, 0
    x = fx.Float8Tensor(c, torch.tensor([0.25]))
    assert x.dtype == torch.bfloat16 and x.scale_dim is None
    assert x.dequantize(torch.float32).tolist() == [[0.25, -0.25], [0.5, 0.0]]


@pytest.mark.parametrize("how", ["t", "transpose", "transpose_neg", "permute", "T"])
def test_relayouts_keep_the_codes(how):
    x = fx.Float8Tensor(codes_4x16(F4), torch.linspace(0.5, 2, 4), 0, torch.float32)
    y = {"t": lambda: x.t(), "transpose": lambda: x.transpose(0, 1), "transpose_neg": lambda: x.transpose(-1, -2),
         "permute": lambda: x.permute(1, 0), "T": lambda: x.T}[how]()
    assert isinstance(y, fx.Float8Tensor) and y.shape == (16, 4) and y.scale_dim == 1
    assert y.codes.data_ptr() == x.codes.data_ptr()
    assert torch.equal(y.dequantize(), x.dequantize().t())
    assert y.t().scale_dim == 0


def test_alias_copy_and_fallback():
    x = fx.Float8Tensor(codes_4x16(), torch.tensor([2.0]), None, torch.float32)
    d = x.detach()
    assert isinstance(d, fx.Float8Tensor) and d.codes.data_ptr() == x.codes.data_ptr()
    c = x.clone()
    assert isinstance(c, fx.Float8Tensor) and c.codes.data_ptr() != x.codes.data_ptr()
    assert torch.equal(c.dequantize(), x.dequantize())
    y = x * 2 + 1  # any other operation dequantizes and runs in the nominal dtype
    assert type(y) is torch.Tensor and torch.equal(y, x.dequantize() * 2 + 1)
    z = x.reshape(8, 8)  # a reshape is not a pure transpose: dequantized
    assert type(z) is torch.Tensor and torch.equal(z, x.dequantize().reshape(8, 8))


def test_products_that_cannot_use_the_library_dequantize():
    """K not a multiple of 16 and a scale that varies along K run on the dequantized values (CPU here:
    such products never reach the library)."""
    a = fx.Float8Tensor(torch.ones(4, 8, dtype=torch.uint8).view(F8), torch.tensor([1.0]), None, torch.float32)
    out = a @ torch.ones(8, 3)
    assert type(out) is torch.Tensor and torch.equal(out, a.dequantize() @ torch.ones(8, 3))
    w = fx.Float8Tensor(codes_4x16(), torch.linspace(1, 2, 16), 1, torch.float32)  # per column = along K of w @ x
    x = torch.randn(16, 5)
    assert torch.equal(w @ x, w.dequantize() @ x)


@pytest.mark.parametrize("kw,exc,text", [
    (dict(lr=-1.0), ValueError, "lr"), (dict(eps=-1e-8), ValueError, "eps"),
    (dict(betas=(0.9, 1.0)), ValueError, "betas"), (dict(betas=(0.9,)), ValueError, "betas"),
    (dict(state_dtype=torch.float16), TypeError, "state_dtype"), (dict(grad_scale=0.0), ValueError, "grad_scale"),
    (dict(fp8_copy=torch.bfloat16), TypeError, "fp8_copy"), (dict(fp8_margin=0.0), ValueError, "fp8_margin"),
])
def test_adamw_rejects(kw, exc, text):
    with pytest.raises(exc, match=text):
        fx.AdamW([torch.nn.Parameter(torch.ones(3))], **kw)


def test_adamw_defaults_match_torch():
    p = [torch.nn.Parameter(torch.ones(3))]
    ours, ref = fx.AdamW(p).defaults, torch.optim.AdamW(p).defaults
    for k in ("lr", "betas", "eps", "weight_decay"):
        assert ours[k] == ref[k], k


def test_rejects_cpu_tensors():
    with pytest.raises(ValueError, match="ROCm device"):
        fx.matmul(torch.zeros(16, 16), torch.zeros(16, 16))
    with pytest.raises(ValueError, match="ROCm device"):
        fx.cast(torch.zeros(16), torch.bfloat16)
