"""The tuner on the GPU (e5m2effma_amd/tune/e5ma_tune --dry-run): it times every candidate of every launch
choice through the library's launchers and reports an entry whose values are among the candidates.
Launch choices never change results: the tuner compares the cast, quantize, half-tile and GEMV-shape candidates'
outputs bit for bit (none may differ), Adam is grid-stride like them, and split-K is held to the same bound by the GEMM
tests with and without it."""
import os
import re
import subprocess

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TUNER = os.path.join(ROOT, "e5m2effma_amd", "tune", "e5ma_tune")


def test_tuner_dry_run():
    assert os.path.exists(TUNER), "tuner not built (make -C e5m2effma_amd/csrc)"
    r = subprocess.run([TUNER, "--dry-run"], capture_output=True, text=True, timeout=300, cwd=ROOT)
    print(r.stdout)
    assert r.returncode == 0, r.stderr
    m = re.search(r'entry: \{"(gfx950)", (\d+), \{(-?\d+), (\d+), (\d+), (\d+), (\d+), (\d+), (\d+)\}\}', r.stdout)
    assert m, r.stdout
    split, cast, abf, af32, quant, tail, rows = map(int, m.groups()[2:])
    assert tail in (0, 1) and rows in (1, 2, 4)
    assert split in (0, 2, 4, 8) and cast in (2048, 4096, 8192, 16384, 32768)
    assert abf in (16384, 32768, 65536, 131072) and af32 in (4096, 8192, 16384, 32768)
    assert quant in (512, 1024, 2048, 4096, 8192, 16384)
    # every cast / quantize candidate produced the same codes, scale_inv and amax, the half-tile GEMMs the same D
    # as the whole-tile ones, and the GEMV row shapes the same y
    assert re.search(r"outputs of 14 cast / quantize / half-tile / GEMV candidates compared with their first "
                     r"candidate's: 0 differ", r.stdout), r.stdout
