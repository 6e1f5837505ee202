"""Runs the C++ drop-in tests (tests/cpp, built by __graft_entry__.build()) on the GPU: the
reference's autograd/tests/test_sgd.cpp known answers, the traced layers' sgd_step surface,
Adam/AdamW against a host restatement, the static layers' and transformer modules'
sgd_step / zero_grad, a train_mlp-style loop whose loss must fall, and the store's data paths
(test_store: uploads/downloads, state records, checkpoint).

Each test also runs as a host-side AddressSanitizer/UBSan build (tests/cpp/build-asan against
tt-perf_amd/lib/asan): any invalid host memory access or undefined behaviour in the library's
host code or the C++ headers fails the run.  Device code is the same in both builds."""
import os
import subprocess

import pytest

from conftest import REPO

pytestmark = pytest.mark.gpu

CPP = os.path.join(REPO, "tests", "cpp")
TESTS = ["test_sgd", "test_traced", "test_adam", "test_modules", "train_mlp", "test_store"]


def _run(exe, env=None):
    p = subprocess.run([exe], capture_output=True, text=True, timeout=240, env=env)
    print(p.stdout[-3000:])
    return p


@pytest.mark.parametrize("name", TESTS)
def test_cpp_dropin(name):
    exe = os.path.join(CPP, "build", name)
    if not os.access(exe, os.X_OK):
        subprocess.run(["make", "-s", "-C", CPP], check=True)
    p = _run(exe)
    assert p.returncode == 0, f"{name} exited {p.returncode}:\n{p.stdout[-3000:]}\n{p.stderr[-2000:]}"
    assert f"{name}: PASS" in p.stdout


def test_gpt2_step_bench_program_at_small_dimensions():
    """tests/cpp/bench_gpt2_step (bench.py's C++ drop-in leg) on a 2-layer GPT model of small
    dimensions: its checks pass (step count and loss scale after the AdamW steps, bf16 weights
    = RNE of the master, an overflow step skipped through autograd::AdamW, sgd_step = w - lr*g)
    and it prints its JSON line.  300 ms of settle steps at this size are usually more than
    2000 steps, so the scale grows on the way (the program checks the scale either way)."""
    import json
    exe = os.path.join(CPP, "build", "bench_gpt2_step")
    if not os.access(exe, os.X_OK):
        subprocess.run(["make", "-s", "-C", CPP], check=True)
    env = dict(os.environ, BENCH_LAYERS="2", BENCH_DIM="128", BENCH_HEADS="4", BENCH_SEQ="64",
               BENCH_VOCAB="1000", BENCH_ITERS="5", BENCH_WARMUP="2", BENCH_SETTLE_MS="300")
    p = _run(exe, env)
    assert p.returncode == 0, f"exited {p.returncode}:\n{p.stdout[-3000:]}\n{p.stderr[-2000:]}"
    assert "bench_gpt2_step: PASS" in p.stdout
    res = json.loads(next(ln for ln in p.stdout.splitlines() if ln.startswith('{"bench"')))
    # 2 embeddings + 2 blocks of 16 tensors + the output projection's weight and bias
    assert res["tensors"] == 36 and res["layers"] == 2
    assert res["params"] == 1000 * 128 + 64 * 128 + 2 * (4 * 128 + 4 * (128 * 128 + 128) +
                                                          2 * 128 * 512 + 512 + 128) + 128 * 1000 + 1000
    assert res["adamw_ms_per_step"] > 0 and res["sgd_ms_per_step"] > 0


@pytest.mark.parametrize("name", TESTS)
def test_cpp_dropin_host_sanitizers(name):
    exe = os.path.join(CPP, "build-asan", name)
    if not os.access(exe, os.X_OK):
        pytest.skip("sanitizer build absent (make -C tt-perf_amd asan && make -C tests/cpp asan)")
    # Leak checking is off: the HIP runtime keeps allocations until exit by design.  The
    # quarantine (freed memory held back to catch use after free) is made larger than these
    # programs ever free, so it never recycles: at exit the HIP runtime's teardown frees its
    # host objects through ASan after the device runtime is gone, and a recycle at that point
    # returns a quarantined device chunk to ASan's device allocator, which aborts ("CHECK
    # failed: sanitizer_allocator_device.h ... dev_runtime_unloaded_") after the program's own
    # checks have passed.  Whether a program hits it depended on how full the quarantine
    # happened to be at exit.
    env = dict(os.environ,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:quarantine_size_mb=16384",
               UBSAN_OPTIONS="print_stacktrace=1")
    p = _run(exe, env)
    assert p.returncode == 0, f"{name} (ASan/UBSan) exited {p.returncode}:\n{p.stdout[-3000:]}\n{p.stderr[-4000:]}"
    assert f"{name}: PASS" in p.stdout
    assert "ERROR: AddressSanitizer" not in p.stderr and "runtime error" not in p.stderr, p.stderr[-4000:]
