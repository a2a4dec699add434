"""The C++ host layer (include/omni_kernel.hpp) driven by a C++ test program,
tests/cpp/test_int8_matmul.cpp, which mirrors the reference's own operator
tests (crates/omni-kernel/src/int8_matmul.rs:700-786) and the prototype's
check shapes (prototypes/int8-gemm/src/main.rs:69-89). __graft_entry__.build()
compiles it; the GPU test runs it."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_int8_matmul")


def test_cpp_driver_is_built():
    assert os.path.exists(BIN), "run __graft_entry__.build() (make -C tests/cpp) first"


@pytest.mark.gpu
def test_cpp_host_layer_on_gpu():
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "OK (0 failures)" in r.stdout
