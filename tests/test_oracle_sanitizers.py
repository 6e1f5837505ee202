"""The CPU oracle (the parity checker) under AddressSanitizer and UBSan: tests/san/oracle_san.c
drives every orc_* entry point on ragged tables with exact-size buffers; the build below
compiles it together with oracle/ttp_oracle.c, instrumented, and any invalid access or
undefined behaviour fails the run.  CPU only."""
import os
import shutil
import subprocess

import pytest

from conftest import REPO


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_oracle_under_asan_and_ubsan(tmp_path):
    exe = tmp_path / "oracle_san"
    cmd = ["gcc", "-std=c11", "-O1", "-g", "-fno-omit-frame-pointer", "-ffp-contract=off",
           "-fopenmp", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-I", os.path.join(REPO, "oracle"),
           os.path.join(REPO, "oracle", "ttp_oracle.c"),
           os.path.join(REPO, "tests", "san", "oracle_san.c"),
           "-lm", "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1", UBSAN_OPTIONS="print_stacktrace=1",
               OMP_NUM_THREADS="4")
    p = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    print(p.stdout[-2000:])
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-4000:]
    assert "oracle_san: PASS" in p.stdout
    assert "runtime error" not in p.stderr, p.stderr[-4000:]
