"""The multiply-and-shift division the kernels use for block_size and
num_kv_heads (voiceagent_amd/csrc/fastdiv.h), checked against integer
division on the host: every divisor up to 4096 over [0, 2^17) and the top of
the range, and large, prime and power-of-two divisors around their multiples
up to 2^31 - 1."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_fastdiv_matches_integer_division(tmp_path):
    exe = tmp_path / "fastdiv_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-o", str(exe),
                    os.path.join(HERE, "native", "fastdiv_check.cpp")], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout + out.stderr
