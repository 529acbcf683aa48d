"""The WO kernel's Q8_0 scale d = amax / 127 without a division instruction
(a multiply by RN(1/127) and one FMA correction, quantize_part in
arclight_amd/csrc/matmul_q4.hip) equals the IEEE quotient that the
reference's quantize_row_q8_0 computes (nnml/src/ops/arm/arm.cpp:1819-1848)
for every finite non-negative float: all 2^31 - 2^23 bit patterns, checked
by tests/csrc/q8_scale_division.c under IEEE single-precision arithmetic
with a fused multiply-add (what v_mul_f32 and v_fma_f32 compute), in 10
processes. The kernel passes an infinite amax through unchanged, as the
division gives it."""
import os
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_scale_division_matches_ieee_for_every_float():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "q8_scale_division")
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-march=x86-64-v3", "-o", exe,
                        os.path.join(HERE, "csrc", "q8_scale_division.c"), "-lm"], check=True)
        # quotients below 2^-126 (x below about 2^-119) are subnormal, which the
        # host's FPU computes slowly: that stretch gets eight of the ten parts
        slow_lo, slow_hi = 0x00800000, 0x10000000
        bounds = [0] + [slow_lo + (slow_hi - slow_lo) * i // 8 for i in range(9)] + [0x7f800000]
        procs = [subprocess.Popen([exe, f"{lo:x}", f"{hi:x}"], stdout=subprocess.PIPE, text=True)
                 for lo, hi in zip(bounds[:-1], bounds[1:])]
        outs = [p.communicate()[0] for p in procs]
        assert all(p.returncode == 0 for p in procs)
        mismatches = sum(int(o.strip().split("\n")[-1]) for o in outs)
        assert mismatches == 0, "".join(outs)
