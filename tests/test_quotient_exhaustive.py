"""Exhaustive CPU check of the fast bf16 quantization arithmetic of the pack
kernel: scale = bf16(amax/127 or amax/7) by constant-reciprocal + fma
correction, and the element quotient x/s by r = RN(1/s) + one fma correction
(Markstein), against correctly rounded division, over every bf16 input of the
domain a row can produce (tests/native/quotient_check.c)."""

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def test_fast_bf16_quotient_is_exact(tmp_path):
    exe = tmp_path / "quotient_check"
    subprocess.check_call(["gcc", "-O2", "-fopenmp", "-ffp-contract=off",
                           os.path.join(HERE, "native", "quotient_check.c"), "-o", str(exe), "-lm"])
    out = subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True, timeout=600)
    print(out.stdout)
    assert out.returncode == 0, out.stdout
    fields = out.stdout.split()
    assert fields[1] == "0" and fields[3] == "0" and fields[5] == "0", out.stdout
    assert int(fields[7]) > 10**9  # every (s, x) pair of the domain was visited
