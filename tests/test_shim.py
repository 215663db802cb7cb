"""The Python layer's host-side behaviour (no GPU): Float8Tensor construction, views and fallbacks,
AdamW argument checks, the dtype alias and the rejection of CPU tensors.  The reference pins the same
behaviour in binds/python/tests/test_e5m2effma.py:254-336."""
import pytest
import torch

import e5m2effma_amd as fx

F8, F4 = torch.float8_e5m2, torch.float8_e4m3fn


def test_dtype_alias():
    assert torch.e5m2effma is torch.float8_e5m2 and fx.e5m2 is torch.float8_e5m2 and fx.e4m3 is torch.float8_e4m3fn


def test_exports():
    for name in ("matmul", "linear", "cast", "adam_step", "AdamW", "Float8Tensor", "quantize_linear_"):
        assert name in fx.__all__ and hasattr(fx, name)


def test_float8tensor_rejects_bad_input():
    d = torch.zeros(4, 16, dtype=F8)
    with pytest.raises(TypeError, match="float8_e5m2"):
        fx.Float8Tensor(d.float(), torch.ones(1))
    with pytest.raises(TypeError, match="float32"):
        fx.Float8Tensor(d, torch.ones(1, dtype=torch.float64))
    with pytest.raises(ValueError, match="scale_dim"):
        fx.Float8Tensor(d, torch.ones(16), 0)
    with pytest.raises(ValueError, match="one element"):
        fx.Float8Tensor(d, torch.ones(2))
    with pytest.raises(TypeError, match="nominal dtype"):
        fx.Float8Tensor(d, torch.ones(1), None, torch.float64)
    with pytest.raises(ValueError, match="ROCm"):
        fx.Float8Tensor.from_float(torch.ones(4, 16))


def test_float8tensor_views_keep_fp8():
    codes = torch.arange(64, dtype=torch.uint8).reshape(4, 16).view(F8)
    s = torch.tensor([0.5, 1.0, 2.0, 4.0])
    x = fx.Float8Tensor(codes, s, 0, torch.float32)
    assert x.shape == (4, 16) and x.dtype == torch.float32 and x._data.dtype == F8
    xt = x.t()
    assert isinstance(xt, fx.Float8Tensor) and xt._scale_dim == 1 and xt.shape == (16, 4)
    assert xt._data.data_ptr() == x._data.data_ptr()
    assert xt.t()._scale_dim == 0 and x.transpose(0, 1)._scale_dim == 1
    assert isinstance(x.detach(), fx.Float8Tensor) and isinstance(x.clone(), fx.Float8Tensor)
    assert x.clone()._data.data_ptr() != x._data.data_ptr()
    ref = codes.float() * s[:, None]
    assert torch.equal(x.float(), ref) and torch.equal(x.dequantize(torch.float32), ref)
    assert x.to(torch.bfloat16).dtype == torch.bfloat16
    y = x * 2  # any other op dequantizes
    assert type(y) is torch.Tensor and torch.equal(y, ref * 2)


def test_float8tensor_per_tensor_scale():
    codes = torch.tensor([0x3C, 0xBC, 0x40, 0x00], dtype=torch.uint8).view(F8).reshape(2, 2)  # 1, -1, 2, 0
    x = fx.Float8Tensor(codes, torch.tensor([0.25]))
    assert x.dtype == torch.bfloat16
    assert x.dequantize(torch.float32).tolist() == [[0.25, -0.25], [0.5, 0.0]]


def test_adamw_rejects_bad_hyperparameters():
    p = [torch.nn.Parameter(torch.ones(3))]
    with pytest.raises(ValueError):
        fx.AdamW(p, lr=-1.0)
    with pytest.raises(ValueError, match="betas"):
        fx.AdamW(p, betas=(0.9, 1.0))
    with pytest.raises(TypeError, match="state_dtype"):
        fx.AdamW(p, state_dtype=torch.float16)


def test_matmul_rejects_cpu_tensor():
    with pytest.raises(ValueError, match="ROCm device"):
        fx.matmul(torch.zeros(16, 16), torch.zeros(16, 16))
    with pytest.raises(ValueError, match="ROCm device"):
        fx.cast(torch.zeros(16), torch.bfloat16)
