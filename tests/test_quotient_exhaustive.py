"""Exhaustive CPU checks of the division-free quotients of the kernels against
correctly rounded division.

The pack kernel: scale = bf16(amax/127 or amax/7) by constant-reciprocal + fma
correction, and the element quotient x/s by r = RN(1/s) + one fma correction
(Markstein), over every bf16 input of the domain a row can produce
(tests/native/quotient_check.c). The denoising-step row kernels: RMSNorm's bf16
x / rs and the INT8Linear activation quantization
(tests/native/step_quotient_check.c)."""

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


def test_step_row_quotients_are_exact(tmp_path):
    """The denoising-step row kernels divide without a division: RMSNorm's
    bf16 x / rs as bf16(x * RN(1/rs)), and the INT8Linear activation
    quantization's x / s by Markstein's correction. Checked against correctly
    rounded division over every bf16 pair of their domains and 10^8 random
    fp32 pairs (tests/native/step_quotient_check.c)."""
    exe = tmp_path / "step_quotient_check"
    subprocess.check_call(["gcc", "-O2", "-fopenmp", "-ffp-contract=off",
                           os.path.join(HERE, "native", "step_quotient_check.c"), "-o", str(exe),
                           "-lm"])
    out = subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True, timeout=600)
    print(out.stdout)
    assert out.returncode == 0, out.stdout
    f = out.stdout.split()
    assert all(f[i] == "0" for i in (1, 3, 5, 7, 9, 15, 17)), out.stdout
    # every pair of the bf16 and fp16 domains visited
    assert int(f[11]) > 6 * 10**8 and int(f[13]) > 10**9 and int(f[19]) > 10**9
