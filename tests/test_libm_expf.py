"""The expf restatement (hessboost_amd/csrc/kernels/libm_expf.h) against the
host C library's expf, the function hessboost's softmax and logistic scalar
rows call through f32::exp (simd/mod.rs:425-427, 580-600): every f32, bit
for bit (NaNs as NaNs)."""
import os
import shutil
import subprocess
import textwrap

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
HEADER = os.path.join(HERE, "..", "hessboost_amd", "csrc", "kernels", "libm_expf.h")

PROGRAM = textwrap.dedent(r"""
    #include <math.h>
    #include <stdio.h>
    #include "libm_expf.h"
    int main(void) {
        uint64_t tab[32];
        for (int i = 0; i < 32; i++) tab[i] = hbr_f64_to_bits(exp2((double)i / 32.0)) - ((uint64_t)i << 47);
        long long bad = 0, n = 0;
    #pragma omp parallel for reduction(+:bad,n) schedule(static)
        for (long long b = 0; b <= 0xFFFFFFFFLL; b += STEP) {
            uint32_t u = (uint32_t)b; float x; memcpy(&x, &u, 4);
            float want = expf(x), got = hbr_expf_libm(x, tab);
            uint32_t uw, ug; memcpy(&uw, &want, 4); memcpy(&ug, &got, 4);
            n++;
            bad += uw != ug && !(want != want && got != got);
        }
        printf("%lld %lld\n", n, bad);
        return 0;
    }
""")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_restated_expf_equals_host_libm_for_every_float(tmp_path):
    src = tmp_path / "expf_check.c"
    src.write_text(PROGRAM)
    exe = tmp_path / "expf_check"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-builtin", "-DSTEP=1",
                    "-I", os.path.dirname(HEADER), "-o", str(exe), str(src), "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    n, bad = int(out[0]), int(out[1])
    assert n == 1 << 32
    assert bad == 0, f"{bad} of {n} inputs differ from the host expf"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_a_plain_rounded_double_exp_is_not_enough(tmp_path):
    """Rounding a correctly rounded f64 exp to f32 differs from the host
    expf on some inputs: the restatement is needed (a mistake in it would
    show up as this many mismatches, not zero)."""
    src = tmp_path / "round_check.c"
    src.write_text(PROGRAM.replace("hbr_expf_libm(x, tab)", "(float)exp((double)x)"))
    exe = tmp_path / "round_check"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-builtin", "-DSTEP=1",
                    "-I", os.path.dirname(HEADER), "-o", str(exe), str(src), "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert int(out[1]) > 0
