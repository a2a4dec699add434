"""fp16 linear: the oracle pinned, the host guards and the C-ABI guard (CPU only)."""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from f16_data import DEPTH_SHAPES, depth_tolerance, depth_w, depth_x
from omni_int8 import _lib
from omni_int8.f16 import depth_try_linear, tensorops_try_linear


def test_f64_truth_matches_numpy(oracle):
    rng = np.random.default_rng(7)
    for rows, k, n in [(1, 32, 5), (3, 96, 17), (7, 256, 33)]:
        x = rng.standard_normal((rows, k)).astype(np.float16)
        w = (rng.standard_normal((n, k)) * 0.1).astype(np.float16)
        got = oracle.f16_linear_f64(x, w)
        ref = x.astype(np.float64) @ w.astype(np.float64).T
        np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_f64_truth_closed_form(oracle):
    for k in (32, 1024):
        x = np.full((2, k), 0.5, dtype=np.float16)
        w = np.full((3, k), -0.25, dtype=np.float16)
        assert np.all(oracle.f16_linear_f64(x, w) == k * 0.5 * -0.25)


def _lane_strided_numpy(x16, w16):
    """metal_depth.rs:13-35 restated in numpy: per lane l, the f32 sum of
    products over k = 32 i + l in order, then lane distances 16 .. 1."""
    x = x16.astype(np.float32)
    w = w16.astype(np.float32)
    rows, k = x.shape
    n = w.shape[0]
    out = np.empty((rows, n), dtype=np.float16)
    for m in range(rows):
        lanes = np.zeros((n, 32), dtype=np.float32)
        for i in range(k // 32):
            lanes += w[:, 32 * i:32 * i + 32] * x[m, 32 * i:32 * i + 32]
        d = 16
        while d >= 1:
            lanes[:, :d] += lanes[:, d:2 * d]
            d //= 2
        out[m] = lanes[:, 0].astype(np.float16)
    return out


def test_gemv_restatement_matches_numpy_order(oracle):
    for rows, k, n in [(1, 32, 7), (2, 96, 65), (3, 1024, 40)]:
        x = depth_x(rows, k).astype(np.float16)
        w = depth_w(k, n).astype(np.float16)
        got = oracle.f16_gemv(x, w)
        assert np.array_equal(got.view(np.uint16), _lane_strided_numpy(x, w).view(np.uint16))


@pytest.mark.parametrize("rows,k,n", DEPTH_SHAPES[:4])
def test_gemv_restatement_within_reference_tolerance(oracle, rows, k, n):
    x = depth_x(rows, k).astype(np.float16)
    w = depth_w(k, n).astype(np.float16)
    expected = oracle.f16_linear_f64(x, w)
    got = oracle.f16_gemv(x, w).astype(np.float64)
    assert np.all(np.abs(got - expected) < depth_tolerance(expected))


def test_host_guards_return_none_off_gpu():
    # crates/breeze-tts/src/metal_depth_tests.rs:83-89: a CPU backend keeps its path
    x = torch.zeros((1, 32), dtype=torch.float16)
    w = torch.zeros((32, 7), dtype=torch.float16)
    assert depth_try_linear(x, w) is None
    x = torch.zeros((256, 4096), dtype=torch.float16)
    w = torch.zeros((4096, 4096), dtype=torch.float16)
    assert tensorops_try_linear(x, w) is None


def test_c_abi_guards():
    L = _lib.lib()
    NH, BAD = _lib.OMNI_NOT_HANDLED, _lib.OMNI_BAD_ARGUMENT
    # metal_depth.rs:94-104: rows 1..=64, k % 32 == 0, 1..=4096 columns
    for rows, n, k in [(0, 7, 32), (65, 7, 32), (1, 7, 48), (1, 0, 32), (1, 4097, 32), (1, 7, 0)]:
        assert L.omni_f16_gemv(None, None, rows, n, k, None, None) == NH, (rows, n, k)
    assert L.omni_f16_gemv(None, None, 64, 4096, 32, None, None) == BAD  # guard passed, null pointers
    # metal_tensorops.rs:174-187: rows 256..=65535, k and n multiples of 64 in 4096..=12288
    for rows, n, k in [(255, 4096, 4096), (65536, 4096, 4096), (256, 4096, 4032), (256, 4160 - 1, 4096),
                       (256, 12352, 4096), (256, 4096, 12352), (256, 4096, 4100)]:
        assert L.omni_f16_gemm(None, None, rows, n, k, None, None) == NH, (rows, n, k)
    assert L.omni_f16_gemm(None, None, 65535, 12288, 12288, None, None) == BAD


def test_tensorops_switch_is_read_from_environment():
    # OMNI_QWEN_TENSOROPS=0 turns the GEMM off (metal_tensorops.rs:165-169)
    # (a fresh process without torch: the switch is read once per process)
    code = ("import ctypes, sys; L = ctypes.CDLL(sys.argv[1]); f = L.omni_f16_gemm; "
            "I = ctypes.c_int64; P = ctypes.c_void_p; f.argtypes = [P, P, I, I, I, P, P]; "
            "print(f(None, None, 256, 4096, 4096, None, None))")
    for value, status in (("0", _lib.OMNI_NOT_HANDLED), ("1", _lib.OMNI_BAD_ARGUMENT)):
        env = dict(os.environ, OMNI_QWEN_TENSOROPS=value)
        out = subprocess.run([sys.executable, "-c", code, _lib.LIB_PATH], env=env,
                             capture_output=True, text=True, check=True)
        assert int(out.stdout.strip()) == status
