"""Write the committed golden fixtures of the palette path.

    python tests/golden/make_golden.py

palette_kats.json
    Data transcribed from the reference's own tests (they cannot run here:
    the reference converter needs its pinned numpy/coremltools stack):
    * pack_lsb: model/tests/test_convert.py:447-479 - codes 0..31 (5-bit) and
      0..15 (6-bit) and the exact little-endian words they pack to.
    * k_major_output_groups: model/tests/test_convert.py:481-511 - a [4, 8]
      matrix in two 4-column palette groups, its two palettes and the
      expected code order after unpacking (k outer, n inner).
workload_draws.json
    The first values of each seeded workload generator, so a change in the
    generator (or in numpy's PCG64 stream) is caught before it silently
    changes every benchmark input.
"""
from __future__ import annotations

import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))


def palette_kats() -> dict:
    dense = [[float(r * 4 + c) for c in range(4)] + [float(100 + r * 4 + c) for c in range(4)]
             for r in range(4)]
    expected_codes = []
    for row in range(4):
        expected_codes += list(range(row * 4, row * 4 + 4)) * 2
    palettes = [[float(v) for v in range(16)] + [0.0] * 16,
                [float(100 + v) for v in range(16)] + [0.0] * 16]
    return {
        "source": "model/tests/test_convert.py:447-511",
        "pack_lsb": [
            {"bits": 5, "codes": list(range(32)),
             "words": [0x8A418820, 0xC5A92839, 0xCA307B9A, 0x38BDAB49, 0xFFBBCDEB]},
            {"bits": 6, "codes": list(range(16)),
             "words": [0x440C2040, 0xA2481C61, 0x3CE34C2C]},
        ],
        "k_major_output_groups": {
            "bits": 5,
            "output_group_width": 4,
            "dense": dense,
            "palettes": palettes,
            "expected_codes": expected_codes,
            "packed_shape": [1, 5],
        },
    }


def workload_draws() -> dict:
    sys.path.insert(0, ROOT)
    import parakeet_wgsl_amd.workloads as wl

    c1 = wl.single_gemm_fp32(0)
    ff = wl.feed_forward_block(0)
    return {
        "single_gemm_fp32_seed0": {
            "x_first8": [float(v) for v in c1.a.reshape(-1)[:8]],
            "codes_first8": [int(v) for v in c1.weight.codes.reshape(-1)[:8]],
            "packed_first4": [int(v) for v in c1.weight.packed.reshape(-1)[:4]],
            "palette_first4": [float(v) for v in c1.weight.palette.reshape(-1)[:4]],
            "bias_first4": [float(v) for v in c1.bias[:4]],
        },
        "feed_forward_seed0": {
            "x_first8_f16_bits": [int(v) for v in ff.x.view("<u2").reshape(-1)[:8]],
            "w1_codes_first8": [int(v) for v in ff.w1.codes.reshape(-1)[:8]],
            "w2_codes_first8": [int(v) for v in ff.w2.codes.reshape(-1)[:8]],
            "w1_palette_f16_bits": [int(v) for v in ff.w1.palette.view("<u2").reshape(-1)[:4]],
        },
    }


def main() -> None:
    with open(os.path.join(HERE, "palette_kats.json"), "w") as f:
        json.dump(palette_kats(), f, indent=1)
        f.write("\n")
    with open(os.path.join(HERE, "workload_draws.json"), "w") as f:
        json.dump(workload_draws(), f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
