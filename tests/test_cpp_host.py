"""The C++ host side (drift_amd/host, libdrift_ops.so) through its own test
program, tests/cpp/test_host.cpp: without a GPU, the shape and type refusals
with the reference's messages and a library refusal surfacing as a
HipException; on the GPU, operations launched through HipOps held to the
oracle's C functions."""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROGRAM = os.path.join(ROOT, "tests", "cpp", "test_host")


def _sources():
    return [os.path.join(ROOT, "tests", "cpp", "test_host.cpp"), os.path.join(ROOT, "tests", "cpp", "comparison.hpp"),
            os.path.join(ROOT, "drift_amd", "host", "drift_ops.cpp"),
            os.path.join(ROOT, "drift_amd", "host", "drift_ops.hpp")]


def _program():
    """The built test program; made here (host code, seconds) when missing or
    older than its sources."""
    stale = not os.path.exists(PROGRAM) or any(
        os.path.getmtime(s) > os.path.getmtime(PROGRAM) for s in _sources())
    if stale:
        subprocess.run(["make", "-C", os.path.join(ROOT, "drift_amd", "host")], check=True)
        subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cpp")], check=True)
    return PROGRAM


def _run(mode):
    result = subprocess.run([_program(), mode], capture_output=True, text=True, timeout=120)
    print(result.stdout)
    assert result.returncode == 0, result.stdout + result.stderr
    assert " 0 failed" in result.stdout


def test_host_checks():
    _run("--checks")


@pytest.mark.gpu
def test_host_on_the_gpu():
    _run("--gpu")
