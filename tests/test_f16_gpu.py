"""fp16 linear parity on the GPU: the Breeze depth GEMV and the Qwen-Image
DiT GEMM (the reference's two fp16 ``try_linear``s).

The bar is the reference's own: |actual - expected| < 0.002 + 0.001 |expected|
against an f64 dot of the same f16 operands
(crates/breeze-tts/src/metal_depth_tests.rs:67-79), and the north_star
relative-error bar (tests/tolerance.py) besides.
"""
import numpy as np
import pytest
import torch

import omni_int8 as oi
import tolerance
from f16_data import DEPTH_SHAPES, PROBE_SHAPES, depth_tolerance, depth_w, depth_x
from omni_int8.f16 import depth_try_linear, tensorops_try_linear

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    assert oi.arch_supported(torch.cuda.current_device()), "device is not gfx950"


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def check(got, expected, what):
    got = np.asarray(got, dtype=np.float64)
    bad = ~(np.abs(got - expected) < depth_tolerance(expected))
    assert not bad.any(), (what, int(bad.sum()), got[bad][:4], expected[bad][:4])
    assert tolerance.rel_err(got, expected) <= tolerance.FP16_REL_TOL, what


def gpu_f64(x16, wt16):
    """f64 truth on the GPU: x [rows, k] f16, wt [k, n] f16 (products exact in f64)."""
    return host(x16.double() @ wt16.double())


@pytest.mark.parametrize("rows,k,n", DEPTH_SHAPES)
@pytest.mark.parametrize("strided,normalize,output_major",
                         [(False, True, True), (True, True, True), (True, False, True),
                          (False, False, False)])
def test_depth_reference_cases(oracle, rows, k, n, strided, normalize, output_major):
    # metal_depth_tests.rs:16-80: strided activations, an RMS-normalised
    # activation from a reduction, and a contiguous [k, n] weight.
    values = torch.from_numpy(depth_x(rows, k).reshape(-1)).cuda()
    if strided:
        x = values.reshape(k, rows // 2, 2).half().permute(1, 2, 0)
    else:
        x = values.reshape(rows // 2, 2, k).half()
    if normalize:
        xf = x.float()
        x = (xf * (xf.square().mean(dim=2, keepdim=True) + 1e-6).sqrt().reciprocal()).half()
    if output_major:
        w = torch.from_numpy(depth_w(k, n)).cuda().half().t()      # [k, n] view of [n, k]
    else:
        i = np.arange(k * n, dtype=np.int64)
        wk = (((i * 13 % 89).astype(np.float32) - 44.0) / np.float32(251.31)).reshape(k, n)
        w = torch.from_numpy(wk).cuda().half()                     # contiguous [k, n]
    got = depth_try_linear(x, w)
    assert got is not None and got.shape == (rows // 2, 2, n) and got.dtype == torch.float16
    xv = host(x.reshape(rows, k).contiguous()).astype(np.float16)
    wv = host(w.t().contiguous()).astype(np.float16)
    expected = oracle.f16_linear_f64(xv, wv)
    check(host(got).reshape(rows, n), expected, (rows, k, n, strided, normalize, output_major))


@pytest.mark.parametrize("k,n", PROBE_SHAPES)
@pytest.mark.parametrize("rows", [1, 2, 4])
def test_depth_probe_shapes(oracle, rows, k, n):
    # prototypes/tts-gemv/src/main.rs:12-40: (batch, tokens) in (1,1) (1,2) (2,1) (2,2)
    x = torch.from_numpy(depth_x(rows, k)).cuda().half()
    w = torch.from_numpy(depth_w(k, n)).cuda().half().t()
    got = depth_try_linear(x, w)
    if n > 4096:  # outside metal_depth.rs:99
        assert got is None
        return
    expected = oracle.f16_linear_f64(host(x), host(w.t().contiguous()))
    check(host(got), expected, (rows, k, n))
    # the restated reference kernel lands in the same tolerance
    ref_kernel = oracle.f16_gemv(host(x), host(w.t().contiguous())).astype(np.float64)
    assert np.all(np.abs(host(got).astype(np.float64) - ref_kernel) <= 0.002 + 0.002 * np.abs(ref_kernel))


@pytest.mark.parametrize("cfg", ["11", "12", "14", "18", "21", "22", "24", "41"])
def test_gemv_every_configuration(oracle, monkeypatch, cfg, knobs):
    # OMNI_F16_GEMV pins one GEMV instantiation (chunks per lane, rows per
    # workgroup): each on ragged shapes up to its widest row (8192 * chunks).
    knobs.set("OMNI_F16_GEMV", cfg)
    widest = 8192 * int(cfg[0])
    for rows, k, n in ((1, widest, 77), (4, widest - 32, 9), (3, 1536, 130), (2, 32, 5)):
        rng = np.random.default_rng(rows + k + n + int(cfg))
        x = torch.from_numpy(rng.standard_normal((rows, k)).astype(np.float16)).cuda()
        w = torch.from_numpy((rng.standard_normal((n, k)) * 0.02).astype(np.float16)).cuda()
        got = depth_try_linear(x, w.t())
        check(host(got), oracle.f16_linear_f64(host(x), host(w)), (cfg, rows, k, n))


@pytest.mark.parametrize("rows,k,n", [(5, 96, 65), (17, 1024, 256), (33, 4096, 1000),
                                      (64, 8192, 4096), (48, 40960, 33), (2, 40960, 50),
                                      (8, 1024, 256), (16, 4096, 1000), (12, 2048, 64),
                                      (6, 3072, 130)])
def test_skinny_rows(oracle, rows, k, n):
    # 5..64 rows (and rows past the GEMV's widest row) run the skinny MFMA kernel.
    rng = np.random.default_rng(rows * 7 + k + n)
    x = torch.from_numpy(rng.standard_normal((rows, k)).astype(np.float16)).cuda()
    w = torch.from_numpy((rng.standard_normal((n, k)) * 0.02).astype(np.float16)).cuda()
    got = depth_try_linear(x, w.t())
    check(host(got), oracle.f16_linear_f64(host(x), host(w)), (rows, k, n))


def test_depth_guard_returns_none():
    x = torch.zeros((65, 32), dtype=torch.float16, device="cuda")
    w = torch.zeros((32, 7), dtype=torch.float16, device="cuda")
    assert depth_try_linear(x, w) is None                                  # rows > 64
    assert depth_try_linear(x[:4, :16], w[:16]) is None                    # k % 32
    assert depth_try_linear(x[:4].float(), w.float()) is None              # not f16
    assert depth_try_linear(x[:4, :16], w) is None                         # k disagrees
    assert depth_try_linear(x[:4], torch.zeros((32, 4097), dtype=torch.float16, device="cuda")) is None


# docs/qwen-image-tensorops.md:55-62 (M x K x N) and the tail-block cases of :70-72
TENSOROPS_SHAPES = [(1024, 4096, 4096), (1024, 4096, 12288), (1024, 12288, 4096),
                    (4096, 4096, 4096), (4096, 4096, 12288), (4096, 12288, 4096),
                    (257, 4096, 4096), (360, 4096, 4096)]


def rand_operands(rows, k, n, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn((rows, k), generator=g, device="cuda").half()
    w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).half()
    return x, w


@pytest.mark.parametrize("rows,k,n", TENSOROPS_SHAPES)
def test_tensorops_shapes(oracle, rows, k, n):
    x, w = rand_operands(rows, k, n, rows + k + n)
    got = tensorops_try_linear(x, w.t())
    assert got is not None and got.shape == (rows, n)
    got_h = host(got)
    check(got_h, gpu_f64(x, w.t()), (rows, k, n))
    # the CPU f64 oracle on a sample of rows, first and last included
    idx = np.unique(np.r_[0, rows - 1, np.linspace(0, rows - 1, 6).astype(int)])
    xs = host(x)[idx]
    check(got_h[idx], oracle.f16_linear_f64(xs, host(w)), ("oracle rows", rows, k, n))


@pytest.mark.parametrize("tile", ["1", "2", "4", "5", "6", "7", "8", "10", "12", "13", "14"])
def test_every_gemm_kernel(oracle, monkeypatch, tile, knobs):
    # OMNI_F16_TILE pins one kernel: tiled 128 x 128 / 64 x 64, ring 256 x 128,
    # 128 x 128, 128 x 256, the 32-element-K-tile rings 256 x 256 and
    # 256 x 128, and the eight-wave rings 256 x 128 and 256 x 256 (32- and
    # 64-element K tiles; waves 64 x 128 or 128 x 64); ragged row counts and a
    # grid smaller than the CUs.
    knobs.set("OMNI_F16_TILE", tile)
    for rows, k, n in ((300, 4096, 4160), (1000, 4160, 4096), (256, 12288, 12288)):
        x, w = rand_operands(rows, k, n, rows * 3 + int(tile))
        got = tensorops_try_linear(x, w.t())
        check(host(got), gpu_f64(x, w.t()), (tile, rows, k, n))


def test_tensorops_guard_returns_none():
    x = torch.zeros((255, 4096), dtype=torch.float16, device="cuda")
    w = torch.zeros((4096, 4096), dtype=torch.float16, device="cuda")
    assert tensorops_try_linear(x, w) is None                              # rows < 256
    x = torch.zeros((256, 4032), dtype=torch.float16, device="cuda")
    assert tensorops_try_linear(x, w[:4032]) is None                       # k < 4096
    x = torch.zeros((256, 4096), dtype=torch.float16, device="cuda")
    assert tensorops_try_linear(x, w[:, :4000]) is None                    # n % 64


def test_weight_layouts_agree_bitwise():
    # a [k, n] weight stored output-major and one stored [k, n]-contiguous run
    # the same kernel on the same values
    x, w = rand_operands(512, 4096, 4096, 5)
    a = tensorops_try_linear(x, w.t())
    b = tensorops_try_linear(x, w.t().contiguous())
    assert torch.equal(a, b)
    xs = x[:8]
    assert torch.equal(depth_try_linear(xs, w.t()), depth_try_linear(xs, w.t().contiguous()))
