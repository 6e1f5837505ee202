"""Runs the C++ drop-in tests (tests/cpp, built by __graft_entry__.build()) on the GPU: the
reference's autograd/tests/test_sgd.cpp known answers, the traced layers' sgd_step surface,
Adam/AdamW against a host restatement, the static layers' and transformer modules'
sgd_step / zero_grad, and a train_mlp-style loop whose loss must fall."""
import os
import subprocess

import pytest

from conftest import REPO

pytestmark = pytest.mark.gpu

BUILD = os.path.join(REPO, "tests", "cpp", "build")


@pytest.mark.parametrize("name", ["test_sgd", "test_traced", "test_adam", "test_modules",
                                  "train_mlp"])
def test_cpp_dropin(name):
    exe = os.path.join(BUILD, name)
    if not os.access(exe, os.X_OK):
        subprocess.run(["make", "-s", "-C", os.path.join(REPO, "tests", "cpp")], check=True)
    p = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(p.stdout[-3000:])
    assert p.returncode == 0, f"{name} exited {p.returncode}:\n{p.stdout[-3000:]}\n{p.stderr[-2000:]}"
    assert f"{name}: PASS" in p.stdout
