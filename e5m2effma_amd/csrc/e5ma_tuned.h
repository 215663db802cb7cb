// e5ma_tuned.h -- written by the tuner (e5m2effma_amd/tune/tune.cpp; make -C e5m2effma_amd/csrc tune-run):
// per-device launch choices of struct Tuning (e5ma_host.hpp), one entry per (architecture, CU count):
// {arch, cus, {splitk_div, cast_grid, adam_grid_bf16, adam_grid_fp32, quant_grid, tail_half, gemv_rows}}.
// Re-running the tuner on a device adds or replaces that device's entry and keeps the others.
#pragma once
#define E5MA_TUNED_ENTRIES \
  {"gfx950", 256, {4, 32768, 131072, 32768, 512, 0, 2}}, /* entry arch=gfx950 cus=256 tuned on AMD Instinct MI355X */ \

