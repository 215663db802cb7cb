"""The tuner's table (e5m2effma_amd/csrc/e5ma_tuned.h) without a GPU: the shipped table compiles into the
library's entry type, and the tuner's header writer (e5ma_tune --emit) adds an entry for a new device,
replaces the entry of the same (architecture, CU count) and keeps the others -- the reference's
tune/tune.cu:130-166 keeps other compute capabilities' entries the same way."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "e5m2effma_amd", "csrc")
TUNER = os.path.join(ROOT, "e5m2effma_amd", "tune", "e5ma_tune")
ENTRY = re.compile(r'\{"(\w+)", (\d+), \{(-?\d+), (\d+), (\d+), (\d+), (\d+), (\d+), (\d+)\}\}, /\* entry arch=(\w+) cus=(\d+) ')


def entries(path):
    with open(path) as f:
        return [m.groups()[:9] for m in map(ENTRY.search, f) if m]


def compiles(path, tmp_path, count):
    src = tmp_path / "t.cpp"
    src.write_text('struct Tuning { int splitk_div = 4, cast_grid = 8192, adam_grid_bf16 = 65536, adam_grid_fp32 = 8192, '
                   'quant_grid = 8192, tail_half = 1, gemv_rows = 2; };\n'
                   'struct TunedEntry { const char *arch; int cus; Tuning t; };\n'
                   f'#include "{path}"\n'
                   'static const TunedEntry kTuned[] = {E5MA_TUNED_ENTRIES{nullptr, 0, {}}};\n'
                   f'static_assert(sizeof(kTuned) / sizeof(kTuned[0]) == {count + 1}, "entries");\n'
                   'int main() { return kTuned[0].cus > 0 ? 0 : 1; }\n')
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", str(src)], capture_output=True, text=True)
    return r.returncode == 0, r.stderr


def test_shipped_table_has_gfx950_and_compiles(tmp_path):
    path = os.path.join(CSRC, "e5ma_tuned.h")
    es = entries(path)
    assert any(e[0] == "gfx950" and e[1] == "256" for e in es)
    ok, err = compiles(path, tmp_path, len(es))
    assert ok, err


@pytest.mark.skipif(not os.path.exists(TUNER), reason="tuner not built (make -C e5m2effma_amd/csrc)")
def test_emit_adds_replaces_and_keeps(tmp_path):
    h = tmp_path / "tuned.h"
    shutil.copy(os.path.join(CSRC, "e5ma_tuned.h"), h)
    before = entries(h)
    run = lambda *a: subprocess.run([TUNER, "--emit", str(h), *map(str, a)], check=True, capture_output=True, env={})
    run("gfx942", 304, 2, 4096, 32768, 8192, 4096, 0, 1, "another device")
    es = entries(h)
    assert es[:len(before)] == before and es[-1] == ("gfx942", "304", "2", "4096", "32768", "8192", "4096", "0", "1")
    run("gfx950", 256, 8, 16384, 131072, 4096, 2048, 1, 4, "MI355X")
    es = entries(h)
    assert ("gfx942", "304", "2", "4096", "32768", "8192", "4096", "0", "1") in es
    assert [e for e in es if e[:2] == ("gfx950", "256")] == [("gfx950", "256", "8", "16384", "131072", "4096", "2048", "1", "4")]
    ok, err = compiles(str(h), tmp_path, len(es))
    assert ok, err
