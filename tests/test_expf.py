"""The kernels' expf (c0ven_amd/csrc/device_math.h, compiled for the host from the same source) against libm's expf.

The CPU path computes softmax, the shared gate's sigmoid and SiLU with std::exp (core/cpu/experts.cpp:21-27;
docs/spec/MODEL_LAYER.md:414-449), which on the x86-64 host is glibc's FMA expf. The restatement must give its bits
on every input, so the check is exhaustive (all 2^32 floats, OpenMP); the GPU parity tests then see the same bits
end to end (softmax weights, shared gate and SwiGLU outputs bit-exact to the oracle, which calls libm).
"""
import os
import subprocess

import pytest

from tests import harness as h

SRC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "expf_check.cpp")


@pytest.fixture(scope="module")
def expf_check(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("expf") / "expf_check")
    subprocess.run(["/opt/rocm/bin/hipcc", "-O2", "-std=c++17", "-fopenmp", "-ffp-contract=off", "-march=x86-64-v3",
                    SRC, "-o", exe], check=True, capture_output=True)
    return exe


def test_expf_restatement_equals_libm_on_all_floats(expf_check):
    r = subprocess.run([expf_check, "1"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0 checked 4294967296" in r.stdout


def test_oracle_expf_is_libm():
    import math
    for x in [-87.5, -10.25, -1.0, -1e-8, 0.0, 1e-8, 0.5, 1.0, 10.0, 88.0]:
        assert h.orc_expf(x) == pytest.approx(math.exp(x), rel=1e-7)
