"""The device HQQ quantizer's powf (lightx2v-rs_amd/csrc/powf_arm.hpp)
against the host libm's powf, which is what the reference's `f32::powf`
calls (crates/lightx2v-core/src/quant.rs:261) and what the oracle calls.

The header is compiled for the host with g++ (the same source the HIP
kernel includes) and swept over f32 arguments; results must be identical
bit for bit.  A double pow rounded once to f32 differs from the libm for
~0.06% of these arguments, so the sweep would catch a restatement that
only approximated the published algorithm.
"""

import os
import subprocess
import tempfile

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "lightx2v-rs_amd", "csrc")

SRC = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "powf_arm.hpp"
using namespace lx2v::powf_arm;
// argv: y, first bits, last bits (exclusive), stride
int main(int argc, char **argv) {
    const float y = strtof(argv[1], 0);
    const long lo = atol(argv[2]), hi = atol(argv[3]), step = atol(argv[4]);
    long n = 0, bad = 0, dbl_bad = 0;
#pragma omp parallel for reduction(+ : n, bad, dbl_bad) schedule(static, 4096)
    for (long u = lo; u < hi; u += step) {
        const float x = u2f((uint32_t)u);
        const float g = powf(x, y);
        if (!isfinite(g) || fabsf(g) < 0x1p-126f || fabs((double)y * log2((double)x)) >= 120.0) continue;
        n++;
        if (f2u(powf_pos(x, y)) != f2u(g)) bad++;
        if (f2u((float)pow((double)x, (double)y)) != f2u(g)) dbl_bad++;
    }
    printf("%ld %ld %ld\n", n, bad, dbl_bad);
    return 0;
}
"""


@pytest.fixture(scope="module")
def sweep():
    d = tempfile.mkdtemp()
    src, exe = os.path.join(d, "sweep.cpp"), os.path.join(d, "sweep")
    with open(src, "w") as f:
        f.write(SRC)
    subprocess.run(["g++", "-O2", "-std=c++17", "-fopenmp", "-ffp-contract=off", "-I", CSRC, src, "-o", exe,
                    "-lm"], check=True)

    def run(y, lo, hi, step):
        out = subprocess.run([exe, repr(float(y)), str(lo), str(hi), str(step)], check=True,
                             capture_output=True, text=True).stdout.split()
        return tuple(int(v) for v in out)

    return run


def test_exp2_table_from_definition():
    """Entry j of the exp2 table is bits(RN(2^(j/32))) - (j << 47)."""
    from decimal import Decimal, getcontext

    getcontext().prec = 60
    text = open(os.path.join(CSRC, "powf_arm.hpp")).read()
    body = text[text.index("#define LX2V_POWF_EXP2_TAB"):]
    body = body[body.index("{") + 1:body.index("}")]
    tab = [int(t.strip().rstrip("ull"), 16) for t in body.replace("\\", "").split(",")]
    assert len(tab) == 32
    for j in range(32):
        v = float(Decimal(2) ** (Decimal(j) / Decimal(32)))  # correctly rounded
        bits = int(np.array([v], np.float64).view(np.uint64)[0])
        assert tab[j] == bits - (j << 47), j


def test_log2_table_consistent():
    """logc = log2(c) with c = 1/invc: each pair agrees with the double
    log2 of its own invc to < 2^-50 (a mistyped digit in either column
    fails this)."""
    import math

    text = open(os.path.join(CSRC, "powf_arm.hpp")).read()
    body = text[text.index("#define LX2V_POWF_LOG2_TAB"):text.index("#define LX2V_POWF_EXP2_TAB")]
    toks = body[body.index("{"):].replace("\\", "").replace("{", " ").replace("}", " ").replace(",", " ").split()
    vals = [float.fromhex(t) for t in toks if t.startswith(("0x", "-0x"))]
    pairs = list(zip(vals[0::2], vals[1::2]))
    assert len(pairs) == 16
    for invc, logc in pairs:
        assert abs(-math.log2(invc) - logc) < 2.0 ** -50, (invc, logc)


def test_hqq_exponent_every_f32(sweep):
    """y = 0.7f - 1.0f (the HQQ shrink): every positive f32, subnormals
    included, identical to the libm."""
    y = np.float32(np.float32(0.7) - np.float32(1.0))
    n, bad, dbl_bad = sweep(y, 1, 0x7F800000, 1)
    assert n > 2_000_000_000
    assert bad == 0, f"{bad} of {n} arguments differ from the libm powf"
    assert dbl_bad > 0  # the sweep can tell the libm from a correctly rounded pow


@pytest.mark.parametrize("y", [0.5, 2.3, -1.7, 0.7, 3.0])
def test_other_exponents_sampled(sweep, y):
    n, bad, _ = sweep(np.float32(y), 1, 0x7F800000, 97)
    assert n > 1_000_000
    assert bad == 0, f"y={y}: {bad} of {n} arguments differ from the libm powf"
