"""The kernels' device code for gfx950 holds no packed FP32 instruction
(v_pk_fma_f32, v_pk_mul_f32, v_pk_add_f32): the build switches them off,
and this compiles every kernel source to assembly and looks."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not os.path.exists(HIPCC) or shutil.which("make") is None, reason="needs hipcc and make")
def test_no_packed_fp32_instructions():
    run = subprocess.run(["make", "-s", "-j4", "-C", os.path.join(ROOT, "drift_amd", "csrc"), "check-isa"],
                         capture_output=True, text=True, timeout=600)
    assert run.returncode == 0, run.stdout[-2000:] + run.stderr[-2000:]
