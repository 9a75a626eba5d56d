"""The FT kernels' index arithmetic (csrc/index_math.h: magic-number division,
the XCD tile schedule, the tile column maps, the long-segment rule) built as
host C++ with the address and undefined-behaviour sanitizers, and checked
against independent formulations (tests/cpu/index_math_test.cpp)."""

import os
import shutil
import subprocess

import pytest

from conftest import ROOT

SRC = os.path.join(ROOT, "tests", "cpu", "index_math_test.cpp")
INC = os.path.join(ROOT, "stockfish-trainer_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_index_math_under_sanitizers(tmp_path):
    exe = str(tmp_path / "index_math_test")
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-Wall", "-Wextra", "-Werror", "-I", INC, SRC, "-o", exe], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert "all checks passed" in r.stdout
