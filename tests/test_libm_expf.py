"""The router's exp (qwen3x_amd/csrc/libm_expf.h) against the host libm's
expf, bit for bit, on every float in [-110, 0] and [0, 88) -- the values the
reference router's std::exp sees (engine.cpp:383-386) are logit - max <= 0.
The header is compiled for the host by hipcc, as the device build compiles it,
and the check runs on the CPU."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc absent")
    exe = str(tmp_path_factory.mktemp("expf") / "libm_expf_check")
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-pthread", "-I", os.path.join(ROOT, "qwen3x_amd", "csrc"),
                    "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "native", "libm_expf_check.cpp"),
                    "-o", exe], check=True)
    return exe


def run(exe, *ranges):
    out = subprocess.run([exe, *[hex(v) for v in ranges]], capture_output=True, text=True, timeout=600)
    return out.returncode, out.stdout.strip()


def test_every_nonpositive_float_down_to_minus_110(checker):
    # -0.0 (0x80000000) through -110.0 (0xc2dc0000), and +0.0.
    rc, text = run(checker, 0x80000000, 0xC2DC0000, 0, 0)
    assert rc == 0, text
    assert text.startswith("checked 1121714178 mismatches 0"), text


def test_every_positive_float_below_88(checker):
    rc, text = run(checker, 1, 0x42AFFFFF)
    assert rc == 0, text


def test_specials(checker):
    # -inf and every float below -110 give +0; NaNs propagate (not compared).
    rc, text = run(checker, 0xC2DC0001, 0xFF800000)
    assert rc == 0, text
