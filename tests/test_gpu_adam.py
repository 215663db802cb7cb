"""e5ma_adam on the GPU, bit-exact against the oracle over several steps (reference
src/adamw_e5m2effma.cu:17-25, 61-96; host scalars :150-157; the reference's own test compares bit for
bit with a host emulation, tests/test_adamw.cu:29-61)."""
import itertools

import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle

pytestmark = pytest.mark.gpu
F32, B16, F16, E5, E4 = oracle.FP32, oracle.BF16, oracle.FP16, oracle.E5M2, oracle.E4M3


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


COMBOS = list(itertools.product([F32, B16], [F32, B16, F16], [F32, B16]))


@pytest.mark.parametrize("pdt,gdt,mdt", COMBOS)
def test_adam_dtype_combinations(dev, pdt, gdt, mdt):
    rng = np.random.default_rng(pdt * 100 + gdt * 10 + mdt)
    qdt = E5 if (pdt + gdt + mdt) % 2 else E4
    assert gu.adam_matches(dev, rng, 100003, pdt, gdt, mdt, qdt=qdt, steps=3)


@pytest.mark.parametrize("offset", [1, 3])
def test_adam_unaligned(dev, offset):
    rng = np.random.default_rng(offset)
    assert gu.adam_matches(dev, rng, 4099, B16, B16, B16, qdt=E5, steps=2, offset=offset)
    assert gu.adam_matches(dev, rng, 4099, F32, F16, F32, qdt=None, steps=2, offset=offset)


@pytest.mark.parametrize("cfg", [
    dict(lr=1e-2, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.1, adamw=0, bias_correction=1, grad_scale=1.0),
    dict(lr=1e-3, beta1=0.8, beta2=0.99, eps=1e-6, weight_decay=0.0, adamw=1, bias_correction=0, grad_scale=0.0),
    dict(lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, adamw=1, bias_correction=1, grad_scale=1024.0),
])
def test_adam_configurations(dev, cfg):
    rng = np.random.default_rng(5)
    assert gu.adam_matches(dev, rng, 70001, F32, F32, F32, qdt=E4, steps=4, cfg=cfg)
    assert gu.adam_matches(dev, rng, 70001, B16, B16, B16, qdt=E5, steps=4, cfg=cfg)


def test_adam_config5_ten_steps(dev):
    """BASELINE config 5 settings (lr 1e-4, betas 0.9 / 0.999, eps 1e-8, wd 0.01, AdamW, 10 steps, E5M2 copy)
    on 1M elements of both state variants."""
    cfg = dict(lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, adamw=1, bias_correction=1,
               grad_scale=1.0)
    rng = np.random.default_rng(10)
    assert gu.adam_matches(dev, rng, 1 << 20, F32, F32, F32, qdt=E5, steps=10, cfg=cfg)
    assert gu.adam_matches(dev, rng, 1 << 20, B16, B16, B16, qdt=E5, steps=10, cfg=cfg)


def test_adam_small_counts(dev):
    rng = np.random.default_rng(6)
    for n in (1, 7, 8, 9, 257):
        assert gu.adam_matches(dev, rng, n, B16, F32, B16, qdt=E4, steps=2)
