"""Writes tests/golden/quant_kats.json: the known-answer data the reference's
own tests and published runs hold for the quantized-linear path.

Every vector below is data copied from a reference test assertion or a
reference run's printed output (source file:line beside it), or derived by
hand from the reference's formula where noted.  Nothing here executes the
reference.  Run: python tests/golden/make_golden.py
"""

import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))

E4M3_ENCODE = [  # crates/lightx2v-core/src/quant.rs:530-534
    (0.0, 0x00, "quant.rs:530"),
    (1.0, 0x38, "quant.rs:531"),
    (-1.0, 0xB8, "quant.rs:532"),
    (448.0, 0x7E, "quant.rs:533"),
    (2.0, 0x40, "quant.rs:534"),
]

E4M3_DECODE = [  # crates/lightx2v-core/src/quant.rs:535-537 (value, tolerance)
    (0x38, 1.0, 1e-7, "quant.rs:535"),
    (0x40, 2.0, 1e-7, "quant.rs:536"),
    (0x01, 2.0**-9 / 8.0, 1e-9, "quant.rs:537"),
]

# f32_to_e4m3 on inputs inside and around the exponent-wrap region
# (quant.rs:396-405: `(e + 7) as u8` wraps for e in {-9, -8, -7} and `exp << 3`
# drops bits), each hand-derived from the reference's formula.
E4M3_ENCODE_DERIVED = [
    (1.0625, 0x39, "tie at mantissa 0.5 rounds away from zero (f32::round)"),
    (2.0**-6, 0x08, "smallest exponent-1 value"),
    (0.9 * 2.0**-6, 0x06, "e=-7: exp wraps to 0, mant round(0.8*8)=6"),
    (2.0**-7, 0x00, "e=-7, mant 0 -> 0x00"),
    (1.9 * 2.0**-8, 0xFF, "e=-8: exp 255, (255<<3)&0xFF=0xF8 | mant 7 -> NaN code"),
    (1.99 * 2.0**-8, 0x7E, "e=-8: mant rounds to 8, exp>=15 -> 0x7E"),
    (1.5 * 2.0**-9, 0xF4, "e=-9: exp 254, (254<<3)&0xFF=0xF0 | 4 -> -192"),
    (2.0**-10, 0x04, "e=-10 < -9: round(a*4096)=4"),
]

CHECK_QUANT = {  # crates/lightx2v-model/src/check.rs:294-320, printed by docs/benchmarks.md:268
    "seed": 17,
    "rows": 8,
    "cols": 256,
    "uniform_a": 1.0,
    "q4_group": 64,
    "hqq": True,
    "printed": "6.552e-2",
    "tolerance": 0.2,
    "src": "check.rs:294-320; docs/benchmarks.md:268 (PASS quant q8/q4/fp8 roundtrip max_abs_err=6.552e-2)",
}

CHECK_LINEAR = {  # crates/lightx2v-model/src/check.rs:74-103, expected values worked by hand
    "x": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0],
    "w": [1.0, 0.0, -1.0, 0.5, 1.0, 0.5, 2.0, -1.0, 0.0, 0.0, 1.0, 2.0],
    "b": [0.5, -0.5, 1.0, 0.0],
    "rows": 2,
    "n": 4,
    "k": 3,
    "want": [-1.5, 3.5, 1.0, 8.0, -1.5, 9.5, 4.0, 17.0],
    "tolerance": 1e-6,
    "src": "check.rs:74-103; docs/benchmarks.md:261 (wgpu max_abs_err=0.000e0)",
}


def main():
    out = {
        "e4m3_encode": [{"v": v, "code": c, "src": s} for v, c, s in E4M3_ENCODE],
        "e4m3_decode": [{"code": c, "value": v, "tol": t, "src": s} for c, v, t, s in E4M3_DECODE],
        "e4m3_encode_derived": [{"v": v, "code": c, "why": s} for v, c, s in E4M3_ENCODE_DERIVED],
        "check_quant": CHECK_QUANT,
        "check_linear": CHECK_LINEAR,
    }
    path = os.path.join(HERE, "quant_kats.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print("wrote", path)


if __name__ == "__main__":
    main()
