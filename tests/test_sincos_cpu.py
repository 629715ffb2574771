"""The rope kernels' double sin and cos (drift_amd/csrc/sincos.hpp: a
three-part pi/2 reduction and fdlibm's kernel polynomials) against the C
library on the CPU, over every angle the kernels make for the runner's rope
bases and widths and random angles of every exponent (tests/cpp/test_sincos.cpp).
The reference takes java.lang.Math's cos and sin of the same float angle
(ops/CpuAttention.scala:124-140); both are within an ulp or two of the exact
value, far below what moves an F32 result."""

import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_sincos_against_the_c_library():
    program = os.path.join(ROOT, "tests", "cpp", "test_sincos")
    source = os.path.join(ROOT, "tests", "cpp", "test_sincos.cpp")
    header = os.path.join(ROOT, "drift_amd", "csrc", "sincos.hpp")
    if not os.path.exists(program) or max(os.path.getmtime(source), os.path.getmtime(header)) > os.path.getmtime(program):
        # only the sin/cos program: the other C++ test links the GPU libraries
        subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cpp"), "sincos"], check=True)
    done = subprocess.run([program], capture_output=True, text=True, timeout=300)
    print(done.stdout)
    assert done.returncode == 0, done.stdout + done.stderr
    assert "worst 2 ulp" in done.stdout or "worst 1 ulp" in done.stdout
