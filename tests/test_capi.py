"""The C-ABI library loads and exports what include/omni_int8.h declares (CPU only).

No kernel runs here: the calls below stop at argument checks or at the
device gate, both of which return before any launch.
"""
import ctypes
import os
import re

import pytest

from omni_int8 import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "omni_int8.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(omni_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    handle = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared_functions():
        assert hasattr(handle, name), name


def test_library_has_no_oracle_dependency():
    # The product library must not link the CPU oracle.
    with open(_lib.LIB_PATH, "rb") as f:
        blob = f.read()
    assert b"oracle_" not in blob
    assert b"liboracle_int8" not in blob


def test_try_int8_gemm_shape_guard_returns_none_status():
    L = _lib.lib()
    ws = L.omni_try_int8_gemm_workspace_size(2, 8)
    assert ws >= 2 * 8 + 8 + 8
    # width % 4 != 0 (int8_matmul.rs:519)
    st = L.omni_try_int8_gemm(None, 0, 2, 6, None, 3, None, 2, None, 2, None, None, ws, None)
    assert st == _lib.OMNI_NOT_HANDLED
    # packed length disagrees with columns * width / 4
    st = L.omni_try_int8_gemm(None, 0, 2, 8, None, 3, None, 2, None, 2, None, None, ws, None)
    assert st == _lib.OMNI_NOT_HANDLED
    # zero-point length disagrees
    st = L.omni_try_int8_gemm(None, 0, 2, 8, None, 4, None, 2, None, 3, None, None, ws, None)
    assert st == _lib.OMNI_NOT_HANDLED
    assert "shapes disagree" in _lib.last_error()


def test_bad_arguments_are_rejected_before_any_launch():
    L = _lib.lib()
    assert L.omni_w8a8_gemm(None, None, None, None, None, None, None, -1, 4, 16, None, 0, None,
                            0, None) == _lib.OMNI_BAD_ARGUMENT
    assert L.omni_w8a8_gemm(None, None, None, None, None, None, None, 1, 4, 16, None, 7, None,
                            0, None) == _lib.OMNI_BAD_ARGUMENT
    assert L.omni_w8a8_gemm(None, None, None, None, None, None, None, 1, 4, 16, None, 0, None,
                            9, None) == _lib.OMNI_BAD_ARGUMENT
    assert L.omni_int8_quantize_rows(None, 5, 1, 16, 16, None, None, None, None) == _lib.OMNI_BAD_ARGUMENT
    assert L.omni_w8a16_gemm(None, None, None, None, 1, 4, 24, None, None) == _lib.OMNI_NOT_HANDLED


def test_lowering_gate(monkeypatch):
    L = _lib.lib()
    monkeypatch.delenv("OMNI_INT8_FORCE_SCALAR", raising=False)
    monkeypatch.delenv("OMNI_CONVROT_TENSOROPS", raising=False)
    assert L.omni_w8a8_lowering(4096) == _lib.OMNI_LOWERING_MFMA
    assert L.omni_w8a8_lowering(36) == _lib.OMNI_LOWERING_SCALAR
    # the reference's switch (int8_tensorops.rs:15-20), read on every call
    monkeypatch.setenv("OMNI_CONVROT_TENSOROPS", "0")
    assert L.omni_w8a8_lowering(4096) == _lib.OMNI_LOWERING_SCALAR
    monkeypatch.setenv("OMNI_CONVROT_TENSOROPS", "1")
    assert L.omni_w8a8_lowering(4096) == _lib.OMNI_LOWERING_MFMA
    monkeypatch.delenv("OMNI_CONVROT_TENSOROPS")
    monkeypatch.setenv("OMNI_INT8_FORCE_SCALAR", "1")
    assert L.omni_w8a8_lowering(4096) == _lib.OMNI_LOWERING_SCALAR


def test_device_gate_without_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; the gate is exercised by the GPU tests")
    L = _lib.lib()
    assert L.omni_int8_arch_supported(0) == 0
    # a valid call shape with no device stops at the gate
    dummy = ctypes.create_string_buffer(64)
    p = ctypes.cast(dummy, ctypes.c_void_p)
    st = L.omni_int8_quantize_rows(p, 0, 1, 4, 4, p, p, p, None)
    assert st == _lib.OMNI_NO_DEVICE


def test_tuning_knobs_set_unset_restore():
    # omni_int8_set_tuning: modes 0 (environment), 1 (unset), 2 (value); an
    # unknown name or mode is rejected; no GPU is involved.
    L = _lib.lib()
    for name in (b"OMNI_W8A8_TILE", b"OMNI_W8A16_SKINNY_SPLIT", b"OMNI_F16_TILE"):
        assert L.omni_int8_set_tuning(name, 2, 17) == _lib.OMNI_OK
        assert L.omni_int8_set_tuning(name, 1, 0) == _lib.OMNI_OK
        assert L.omni_int8_set_tuning(name, 0, 0) == _lib.OMNI_OK
    assert L.omni_int8_set_tuning(b"OMNI_NOT_A_KNOB", 2, 1) == _lib.OMNI_BAD_ARGUMENT
    assert "unknown knob" in _lib.last_error()
    assert L.omni_int8_set_tuning(b"OMNI_W8A8_TILE", 3, 1) == _lib.OMNI_BAD_ARGUMENT
    assert L.omni_int8_set_tuning(None, 2, 1) == _lib.OMNI_BAD_ARGUMENT


def test_no_getenv_on_launch_paths():
    # The kernels' tuning knobs are read from the environment once per
    # process (omni::knob); the only per-call reads are the reference's own
    # switch OMNI_CONVROT_TENSOROPS (int8_tensorops.rs:15-20) and its
    # companion OMNI_INT8_FORCE_SCALAR, plus OMNI_QWEN_TENSOROPS, read once.
    csrc = os.path.join(ROOT, "omni-rs_amd", "csrc")
    found = []
    for name in sorted(os.listdir(csrc)):
        text = open(os.path.join(csrc, name)).read()
        found += [(name, arg) for arg in re.findall(r"getenv\(([^)]*)\)", text)]
    assert sorted(found) == sorted([("capi.hip", '"OMNI_CONVROT_TENSOROPS"'),
                                    ("capi.hip", '"OMNI_INT8_FORCE_SCALAR"'),
                                    ("capi.hip", '"OMNI_QWEN_TENSOROPS"'),
                                    ("capi.hip", "kKnobNames[i]")]), found
