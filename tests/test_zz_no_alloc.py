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


def _into(L, fn, x, code, packed, scale, zero, out):
    """One entry-point call into a preallocated output, no synchronisation
    (capturable)."""
    rows, width = x.shape
    columns = scale.numel()
    st = fn(_ptr(x), code, rows, width, _ptr(packed), packed.numel(), _ptr(scale), columns, _ptr(zero),
            columns, _ptr(out), _stream())
    assert st == _lib.OMNI_OK, _lib.last_error()


def test_no_alloc_inside_graph_capture():
    # The use the entry point exists for: calls inside HIP graph capture.
    # Two calls captured in one graph (the reference's 256 x 4096 x 12288
    # shape, whose GEMM splits K inside the static array, and a ragged one),
    # after one eager warm-up; the graph replayed three times, each time on
    # new activation values written eagerly before the replay and with the
    # outputs poisoned, every replay checked bit for bit against the
    # workspace entry point run eagerly on the same values.
    L = _lib.lib()
    rng = np.random.default_rng(77)
    cases = [_case(rng, 256, 12288, 4096, np.float16), _case(rng, 300, 1024, 700, np.float32)]
    codes = [_lib.OMNI_F16, _lib.OMNI_F32]
    outs = [torch.empty((c[0].shape[0], c[2].numel()), dtype=torch.float32, device="cuda") for c in cases]
    for c, code, out in zip(cases, codes, outs):  # eager warm-up (scratch looked up)
        _into(L, L.omni_try_int8_gemm_noalloc, c[0], code, c[1], c[2], c[3], out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            for c, code, out in zip(cases, codes, outs):
                _into(L, L.omni_try_int8_gemm_noalloc, c[0], code, c[1], c[2], c[3], out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for replay in range(3):
        for c in cases:
            c[0].copy_(torch.from_numpy(rng.standard_normal(tuple(c[0].shape))).to(c[0].dtype).cuda())
        for out in outs:
            out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for c, code, out in zip(cases, codes, outs):
            want = _with_workspace(L, c[0], code, *c[1:])
            assert torch.equal(out.view(torch.int32), want.view(torch.int32)), (replay, tuple(c[0].shape))


FIRST_CALL_IN_CAPTURE = r"""
import ctypes, sys
import numpy as np, torch
sys.path.insert(0, sys.argv[1])
from omni_int8 import _lib
L = _lib.lib()
rows, width, columns = 200, 2048, 300
rng = np.random.default_rng(5)
x = torch.from_numpy(rng.standard_normal((rows, width)).astype(np.float16)).cuda()
w = torch.from_numpy(rng.integers(-128, 128, (columns, width), dtype=np.int8)).cuda().view(torch.int32).reshape(-1)
s = torch.from_numpy(rng.uniform(0.002, 0.02, columns).astype(np.float32)).cuda()
z = torch.zeros(columns, dtype=torch.int32, device="cuda")
out = torch.empty((rows, columns), dtype=torch.float32, device="cuda")
P = lambda t: ctypes.c_void_p(t.data_ptr())
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
side = torch.cuda.Stream()
with torch.cuda.stream(side):
    with torch.cuda.graph(g, stream=side):
        st = L.omni_try_int8_gemm_noalloc(P(x), _lib.OMNI_F16, rows, width, P(w), w.numel(), P(s), columns, P(z),
                                          columns, P(out), ctypes.c_void_p(side.cuda_stream))
torch.cuda.synchronize()
print("status", st, _lib.last_error() if st else "")
assert st == 0
ws_bytes = L.omni_try_int8_gemm_workspace_size(rows, width)
ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
want = torch.empty_like(out)
for replay in range(2):
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert L.omni_try_int8_gemm(P(x), _lib.OMNI_F16, rows, width, P(w), w.numel(), P(s), columns, P(z), columns,
                                P(want), P(ws), ws_bytes, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), want.view(torch.int32)), replay
print("FIRST_CALL_CAPTURE_OK")
"""


def test_no_alloc_first_call_inside_capture():
    # A fresh process whose very first no-alloc call is made under graph
    # capture, so the per-device scratch lookup (hipGetSymbolAddress) and
    # the gfx950 probe happen during capture; the graph is replayed twice
    # and checked against the workspace entry point.
    import os
    import subprocess
    import sys
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "omni-rs_amd")
    r = subprocess.run([sys.executable, "-c", FIRST_CALL_IN_CAPTURE, pkg], capture_output=True, text=True,
                       timeout=110)
    assert r.returncode == 0 and "FIRST_CALL_CAPTURE_OK" in r.stdout, (r.stdout[-2000:], r.stderr[-2000:])
