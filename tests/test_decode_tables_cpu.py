"""The decode kernel's table build and bit cursor (csrc/cachegen_decode.h),
compiled for the host with g++ and checked against the oracle's decoder
(oracle/cachegen.c) on random CDF rows and byte streams; see
tests/decode_tables_check.cpp."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if not shutil.which("g++") or not shutil.which("gcc"):
        pytest.skip("needs gcc and g++")
    d = tmp_path_factory.mktemp("dectab")
    obj = d / "oracle_cachegen.o"
    exe = d / "decode_tables_check"
    subprocess.run(["gcc", "-O2", "-c", os.path.join(REPO, "oracle", "cachegen.c"), "-o", str(obj)], check=True)
    # Built with AddressSanitizer: the lane regions are sized exactly as in
    # the kernel, so a read or write past a lane's region fails the run.
    subprocess.run(["g++", "-O1", "-std=c++17", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    os.path.join(HERE, "decode_tables_check.cpp"), str(obj), "-o", str(exe)], check=True)
    return str(exe)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_decode_tables_match_oracle(checker, seed):
    res = subprocess.run([checker, "3000", str(seed)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.startswith("ok"), res.stdout
