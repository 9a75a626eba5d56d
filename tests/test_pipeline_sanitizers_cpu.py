"""The threaded host pipeline (csrc/host/pipeline.cpp) under the thread sanitizer
and under the address and undefined-behaviour sanitizers: tests/cpu/pipeline_stress.cpp
drives finite, skip-filtered and cyclic streams on 4-6 reader threads,
caller-provided slabs, destruction right after creation, mid-stream and with
slabs held, and a reader failing mid-stream (reported to the consumer, as the
reference's take_error_if_any, src/rust/pipeline.rs:395-410).  Any sanitizer
report fails the test."""

import os
import shutil
import subprocess

import pytest

from conftest import ROOT

SRC = [os.path.join(ROOT, "stockfish-trainer_amd", "csrc", "host", "pipeline.cpp"),
       os.path.join(ROOT, "tests", "cpu", "pipeline_stress.cpp")]
INC = os.path.join(ROOT, "include")

SANITIZERS = {
    "thread": (["-fsanitize=thread"], {"TSAN_OPTIONS": "halt_on_error=1:exitcode=66:second_deadlock_stack=1"}),
    "address,undefined": (["-fsanitize=address,undefined", "-fno-sanitize-recover=all"],
                          {"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0", "UBSAN_OPTIONS": "print_stacktrace=1"}),
}


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
@pytest.mark.parametrize("sanitizer", sorted(SANITIZERS))
def test_pipeline_threads_under_sanitizer(sanitizer, tmp_path):
    flags, env_extra = SANITIZERS[sanitizer]
    exe = str(tmp_path / "pipeline_stress")
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-pthread", *flags, "-Wall", "-Wextra", "-Werror", "-I", INC,
                    *SRC, "-o", exe], check=True)
    r = subprocess.run([exe, str(tmp_path)], capture_output=True, text=True, env=dict(os.environ, **env_extra),
                       timeout=600)
    report = r.stdout[-3000:] + r.stderr[-3000:]
    assert r.returncode == 0, report
    assert "all checks passed" in r.stdout, report
    assert "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, report
