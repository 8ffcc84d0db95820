"""The HardSwish epilogue divides by 6 with a multiply and one fma correction (div6 in
vknn_amd/csrc/kernels/common.h) instead of a full fp32 division. This checks, over all 2^32 fp32
inputs, that the result equals the correctly rounded t / 6 wherever an fp16 store can tell them
apart (the reference's applyAct computes x * clamp(x + 3, 0, 6) / 6 in fp32,
src/backend/cpu/cpu_backend.cpp:33-72)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_div6_exhaustive(tmp_path):
    exe = tmp_path / "div6_check"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", os.path.join(HERE, "div6_check.c"), "-o", str(exe), "-lm"],
                   check=True)
    env = dict(os.environ, OMP_NUM_THREADS=str(min(8, os.cpu_count() or 1)))
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, env=env, timeout=600).stdout.split()
    bad, subnormal = int(out[0]), int(out[1])
    assert bad == 0
    # the differences that remain are confined to subnormal quotients (a few million inputs)
    assert subnormal < (1 << 23)
