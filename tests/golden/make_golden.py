"""Writes the golden vectors of the reference's exact MAC model into tests/golden/.

Source of truth: ``e5ma_ref::lane`` (reference ``tests/e5m2effma_ref.h:114-129``, C entry
``tests/ref_capi.cpp:5``), compiled from the reference sources where they lie into
``oracle/_ref/libref.so`` by ``oracle/Makefile`` (the recipe of the reference ``Makefile:99-100``).
Run in the build container (where /root/reference exists):

    make -C oracle && python tests/golden/make_golden.py

Outputs (data only; nothing of the reference's source text):
  lane_golden.npz   explicit vectors per FP8 pairing: a, b, acc -> RN_BF16(acc + a*b)
  lane_golden.json  the accumulator corpus and SHA-256 digests of the full sweeps
                    (all 65,536 (a, b) pairs x every corpus accumulator, per pairing)
The corpus is the fixed accumulator list of the reference's own checker
(``tests/check_ref.py:71-73``) plus 40 accumulators drawn here from a fixed seed.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402

# reference tests/check_ref.py:71-73 (fixed part of the accumulator corpus)
FIXED_ACCS = [0, 0x8000, 1, 0x8001, 0x7F, 0x807F, 0x80, 0x8080, 0x7F7F, 0xFF7F, 0x7F80, 0xFF80,
              0x7FC0, 0xFFC0, 0x7F81, 0x3F80, 0xBF80, 0x3F81, 0xBF81, 0x3F7F, 0x4380, 0xC380, 0x3B80, 0x3480,
              0x4700, 0xC700, 0x4361, 0x3C00, 0x3800, 0x3700, 0x3680, 0x3600]
# the reference model's format codes: 0 = E4M3, 1 = E5M2 (tests/e5m2effma_ref.h:76)
PAIRINGS = [(1, 1), (1, 0), (0, 1), (0, 0)]
SEED = 0x2545F491  # the reference fixtures' xorshift seed (tests/test_util.h:16), reused as a numpy seed


def corpus():
    rng = np.random.default_rng(SEED)
    extra = rng.integers(0, 0x10000, size=40).tolist()
    return sorted(set(FIXED_ACCS + extra))


def fp8_value(code, fmt):
    return oracle.lib().orc_e5m2_value(int(code)) if fmt else oracle.lib().orc_e4m3_value(int(code))


def sample_cases(rng, fa, fb, n_random=4096, n_near=2048):
    """Random (a, b, acc) triples plus accumulators a few hundred BF16 ulps from the product (the
    cancellation and tie cases of the reference checker, tests/check_ref.py:76-83)."""
    a = rng.integers(0, 256, n_random).astype(np.uint8)
    b = rng.integers(0, 256, n_random).astype(np.uint8)
    acc = rng.integers(0, 0x10000, n_random).astype(np.uint16)
    na, nb, nacc = [], [], []
    while len(na) < n_near:
        x, y = int(rng.integers(0, 256)), int(rng.integers(0, 256))
        px, py = fp8_value(x, fa), fp8_value(y, fb)
        if not (np.isfinite(px) and np.isfinite(py)) or px * py == 0:
            continue
        t = int(oracle.lib().orc_f32_to_bf16(abs(px * py))) + int(rng.integers(-300, 301))
        na.append(x)
        nb.append(y)
        nacc.append((t & 0x7FFF) | (int(rng.integers(0, 2)) << 15))
    return (np.concatenate([a, np.array(na, np.uint8)]), np.concatenate([b, np.array(nb, np.uint8)]),
            np.concatenate([acc, np.array(nacc, np.uint16)]))


def main():
    ref = oracle.ref_library()
    if ref is None:
        sys.exit("oracle/_ref/libref.so is missing: run `make -C oracle` where /root/reference exists")
    accs = np.array(corpus(), np.uint16)
    rng = np.random.default_rng(SEED + 1)
    arrays, digests = {}, {}
    for fa, fb in PAIRINGS:
        tag = f"{fa}{fb}"
        full = oracle.lane_sweep(accs, fa, fb, fn=ref.ref_lane)
        digests[tag] = hashlib.sha256(full.astype("<u2").tobytes()).hexdigest()
        a, b, acc = sample_cases(rng, fa, fb)
        out = np.array([ref.ref_lane(int(x), int(y), int(z), fa, fb) for x, y, z in zip(a, b, acc)], np.uint16)
        arrays[f"a_{tag}"], arrays[f"b_{tag}"], arrays[f"acc_{tag}"], arrays[f"out_{tag}"] = a, b, acc, out
    np.savez_compressed(os.path.join(HERE, "lane_golden.npz"), **arrays)
    with open(os.path.join(HERE, "lane_golden.json"), "w") as f:
        json.dump({"source": "reference tests/e5m2effma_ref.h:114-129 via tests/ref_capi.cpp:5",
                   "format_codes": "0 = E4M3, 1 = E5M2 (pairing key 'fa fb')",
                   "corpus": [int(x) for x in accs], "sweep_layout": "[acc index][a][b], uint16 little-endian",
                   "sha256": digests}, f, indent=1)
    print("wrote", len(accs), "accumulators;", {k: v[:12] for k, v in digests.items()})


if __name__ == "__main__":
    main()
