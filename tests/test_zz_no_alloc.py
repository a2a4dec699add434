"""omni_try_int8_gemm_noalloc against omni_try_int8_gemm, through the C ABI.

The no-allocation entry point keeps its codes, row scales and row sums in a
static device array instead of a caller workspace. Its output must equal the
workspace entry point's bit for bit, on two calls in a row (the second
smaller, so it runs over what the first left in the array), and shapes
beyond the array must be refused before any launch.
"""
import ctypes

import numpy as np
import pytest
import torch

import omni_int8 as oi
from omni_int8 import _lib

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20  # OMNI_NOALLOC_SCRATCH_BYTES in include/omni_int8.h


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _case(rng, rows, width, columns, dtype):
    x = torch.from_numpy(rng.standard_normal((rows, width)).astype(dtype)).cuda()
    w = torch.from_numpy(rng.integers(-128, 128, (columns, width), dtype=np.int8)).cuda()
    scale = torch.from_numpy(rng.uniform(0.002, 0.02, columns).astype(np.float32)).cuda()
    zero = torch.from_numpy(rng.integers(-3, 4, columns).astype(np.int32)).cuda()
    return x, w.view(torch.int32).reshape(-1), scale, zero


def _with_workspace(L, x, code, packed, scale, zero):
    rows, width = x.shape
    columns = scale.numel()
    ws_bytes = L.omni_try_int8_gemm_workspace_size(rows, width)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    out = torch.empty((rows, columns), dtype=torch.float32, device="cuda")
    st = L.omni_try_int8_gemm(_ptr(x), code, rows, width, _ptr(packed), packed.numel(),
                              _ptr(scale), columns, _ptr(zero), columns, _ptr(out), _ptr(ws),
                              ws_bytes, _stream())
    assert st == _lib.OMNI_OK, _lib.last_error()
    torch.cuda.synchronize()
    return out


def _no_alloc(L, x, code, packed, scale, zero):
    rows, width = x.shape
    columns = scale.numel()
    out = torch.full((rows, columns), float("nan"), dtype=torch.float32, device="cuda")
    st = L.omni_try_int8_gemm_noalloc(_ptr(x), code, rows, width, _ptr(packed), packed.numel(),
                                      _ptr(scale), columns, _ptr(zero), columns, _ptr(out),
                                      _stream())
    assert st == _lib.OMNI_OK, _lib.last_error()
    torch.cuda.synchronize()
    return out


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    assert oi.arch_supported(torch.cuda.current_device()), "device is not gfx950"


@pytest.mark.parametrize("dtype,code", [(np.float16, _lib.OMNI_F16), (np.float32, _lib.OMNI_F32)])
def test_no_alloc_matches_workspace_entry_two_calls(dtype, code):
    L = _lib.lib()
    rng = np.random.default_rng(2024)
    # first call: the north-star activation shape (48 MiB of codes), then a
    # smaller ragged one whose rows land on what the first call left behind
    for rows, width, columns in ((4096, 12288, 640), (300, 1024, 700)):
        x, packed, scale, zero = _case(rng, rows, width, columns, dtype)
        want = _with_workspace(L, x, code, packed, scale, zero)
        got = _no_alloc(L, x, code, packed, scale, zero)
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (rows, width, columns)


def test_no_alloc_refuses_shapes_beyond_the_scratch():
    L = _lib.lib()
    rows, width = 8192, 8192  # 64 MiB of codes plus scales and sums: over the limit
    assert L.omni_try_int8_gemm_workspace_size(rows, width) > SCRATCH_BYTES
    columns = 16
    dummy = torch.zeros(16, dtype=torch.int32, device="cuda")
    st = L.omni_try_int8_gemm_noalloc(_ptr(dummy), _lib.OMNI_F16, rows, width, _ptr(dummy),
                                      columns * width // 4, _ptr(dummy), columns, _ptr(dummy),
                                      columns, _ptr(dummy), _stream())
    assert st == _lib.OMNI_BAD_ARGUMENT
    assert "scratch" in _lib.last_error()
    # the reference's shape guard still answers first (None)
    st = L.omni_try_int8_gemm_noalloc(_ptr(dummy), _lib.OMNI_F16, 2, 6, _ptr(dummy), 3,
                                      _ptr(dummy), 2, _ptr(dummy), 2, _ptr(dummy), _stream())
    assert st == _lib.OMNI_NOT_HANDLED
