"""Weight-only int8 (W8A16) parity on the GPU.

The reference has no W8A16 op; its dequantisation convention (w * scale per
output channel, f32 accumulation, int8_matmul.rs:644-649 / quant.rs:186-200)
is restated by the oracle. The bar is the north_star one: max relative error
<= 1e-2 with fp16 output (tests/tolerance.py), against the f64 ground truth
and against the oracle's dequantise-to-f16 route. The fp16-GEMV analog test
of the reference (crates/breeze-tts/src/metal_depth_tests.rs:16-80) sweeps
small and odd shapes the same way.
"""
import numpy as np
import pytest
import torch

import omni_int8 as oi
import tolerance

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    assert oi.arch_supported(torch.cuda.current_device()), "device is not gfx950"


def make(rng, rows, width, columns, bias=False):
    x = rng.standard_normal((rows, width)).astype(np.float16)
    w = rng.integers(-127, 128, (columns, width), dtype=np.int8)
    s = rng.uniform(0.002, 0.02, columns).astype(np.float16)
    b = rng.standard_normal(columns).astype(np.float16) if bias else None
    return x, w, s, b


def gpu_f64_reference(x, w, s, b):
    """Full-size ground truth on the GPU in f64 (products of f16 and int8 are
    exact in f64; the sum carries ~1e-16 relative error)."""
    ref = dev(x).double() @ dev(w).double().T
    ref = ref * dev(s).double()[None, :]
    if b is not None:
        ref = ref + dev(b).double()[None, :]
    return host(ref)


@pytest.mark.parametrize("rows", [1, 2, 3, 4])
@pytest.mark.parametrize("width,columns", [(16, 1), (32, 7), (256, 33), (4096, 100), (4112, 9),
                                          (8192, 1024), (16384, 65)])
def test_gemv_small_and_odd_shapes(oracle, rows, width, columns):
    rng = np.random.default_rng(rows * 31 + width + columns)
    x, w, s, b = make(rng, rows, width, columns, bias=columns % 2 == 1)
    got = host(oi.w8a16_linear(dev(x), dev(w), dev(s), None if b is None else dev(b)))
    ref = oracle.w8a16_f64(x, w, s, b)
    assert tolerance.rel_err(got, ref) <= tolerance.FP16_REL_TOL
    route = oracle.w8a16_gemm(x, w, s, b)
    assert tolerance.rel_err(got, route.astype(np.float64), truth=False) <= tolerance.FP16_REL_TOL


@pytest.mark.parametrize("cfg", ["11", "12", "14", "18", "21", "22", "24",
                                 "142", "144", "124", "182", "242", "222"])
def test_gemv_every_configuration(oracle, monkeypatch, cfg, knobs):
    # OMNI_W8A16_GEMV pins one GEMV instantiation (chunks per lane, rows per
    # batch, and batches per workgroup when there are three digits); each must
    # agree with the oracle on ragged shapes, including the widest row (16384),
    # a row narrower than one wavefront of chunks and column counts that leave
    # the last workgroup's batches partly or wholly past the matrix.
    knobs.set("OMNI_W8A16_GEMV", cfg)
    for rows, width, columns in ((1, 4096, 77), (4, 16384, 9), (3, 1536, 130), (2, 16, 5),
                                 (1, 14336, 31)):
        rng = np.random.default_rng(rows + width + columns + int(cfg))
        x, w, s, b = make(rng, rows, width, columns, bias=rows % 2 == 1)
        got = host(oi.w8a16_linear(dev(x), dev(w), dev(s), None if b is None else dev(b)))
        ref = oracle.w8a16_f64(x, w, s, b)
        assert tolerance.rel_err(got, ref) <= tolerance.FP16_REL_TOL, (cfg, rows, width, columns)


@pytest.mark.parametrize("cfg", ["941", "942", "944", "981", "982", "984"])
def test_gemv_stream_every_configuration(oracle, cfg, knobs):
    # The streamed GEMV (OMNI_W8A16_GEMV=9<rows a batch><workgroups per CU>)
    # on 2..4 activation rows at both K it is built for: ragged column counts
    # (a last batch partly past the matrix), workgroups that take one batch
    # or many, with and without a bias.
    knobs.set("OMNI_W8A16_GEMV", cfg)
    for rows, width, columns in ((2, 4096, 77), (3, 4096, 4099), (4, 4096, 9000), (2, 14336, 31),
                                 (4, 14336, 4097), (3, 14336, 5)):
        rng = np.random.default_rng(rows + width + columns + int(cfg))
        x, w, s, b = make(rng, rows, width, columns, bias=columns % 2 == 1)
        got = host(oi.w8a16_linear(dev(x), dev(w), dev(s), None if b is None else dev(b)))
        ref = oracle.w8a16_f64(x, w, s, b)
        assert tolerance.rel_err(got, ref) <= tolerance.FP16_REL_TOL, (cfg, rows, width, columns)


@pytest.mark.parametrize("rows", [2, 3, 4])
@pytest.mark.parametrize("columns", [1025, 4096, 8191, 14336, 16384])
def test_gemv_stream_default_route(oracle, rows, columns):
    # 2..4 rows at K = 4096 on 4 M to 64 M weights take the streamed GEMV by
    # default.
    rng = np.random.default_rng(rows * 7 + columns)
    x, w, s, b = make(rng, rows, 4096, columns, bias=True)
    got = host(oi.w8a16_linear(dev(x), dev(w), dev(s), dev(b)))
    ref = gpu_f64_reference(x, w, s, b)
    assert tolerance.rel_err(got, ref) <= tolerance.FP16_REL_TOL, (rows, columns)


@pytest.mark.parametrize("width,columns", [(4096, 4099), (14336, 4097), (1536, 8963), (8960, 1539),
                                          (1536, 515), (4096, 1027)])
def test_gemv_k_builds_ragged_columns(oracle, width, columns):
    # One row at K = 4096 / 14336 / 1536 / 8960 runs the GEMV built for that
    # K (one, two or four rows per workgroup by matrix size); column counts
    # leave the last workgroup partly past the matrix.
    rng = np.random.default_rng(width + columns)
    x, w, s, b = make(rng, 1, width, columns, bias=True)
    got = host(oi.w8a16_linear(dev(x), dev(w), dev(s), dev(b)))
    ref = oracle.w8a16_f64(x, w, s, b)
    assert tolerance.rel_err(got, ref) <= tolerance.FP16_REL_TOL, (width, columns)


def test_gemv_exact_on_integer_inputs():
    # integer x, scale 1: every partial sum is an integer below 2^11 -> exact
    x = np.tile(np.arange(-4, 4, dtype=np.float16), (4, 64))[:, :512].copy()
    x = x.reshape(4, 512)
    w = ((np.arange(9 * 512) % 5) - 2).astype(np.int8).reshape(9, 512)
    s = np.ones(9, np.float16)
    got = host(oi.w8a16_linear(dev(x), dev(w), dev(s)))
    want = (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("rows", [1, 4])
@pytest.mark.parametrize("width,columns", [(4096, 4096), (4096, 14336), (14336, 4096),
                                          (4096, 128256)])
def test_config2_decode_sweep_full_size(oracle, rows, width, columns):
    # 7B-LLM decode shapes, M = 1 and 4
    rng = np.random.default_rng(width + columns + rows)
    x, w, s, b = make(rng, rows, width, columns)
    got = host(oi.w8a16_linear(dev(x), dev(w), dev(s)))
    ref = gpu_f64_reference(x, w, s, b)
    assert tolerance.rel_err(got, ref) <= tolerance.FP16_REL_TOL
    cols = rng.choice(columns, 64, replace=False)
    route = oracle.w8a16_gemm(x, w[cols], s[cols])
    assert tolerance.rel_err(got[:, cols], route.astype(np.float64), truth=False) <= tolerance.FP16_REL_TOL


def test_config1_reference_cpu_case(oracle):
    # M=16, K=4096, N=4096, seed 0 (GEMM path at M=16)
    rng = np.random.default_rng(0)
    x, w, s, _ = make(rng, 16, 4096, 4096)
    got = host(oi.w8a16_linear(dev(x), dev(w), dev(s)))
    ref = oracle.w8a16_f64(x, w, s)
    assert tolerance.rel_err(got, ref) <= tolerance.FP16_REL_TOL


@pytest.mark.parametrize("rows,width,columns", [(5, 64, 33), (16, 256, 64), (17, 1536, 1536),
                                                (64, 8960, 1536), (130, 1536, 8960),
                                                (1024, 1536, 2048), (33, 20000, 40)])
def test_mfma_gemm_shapes(oracle, rows, width, columns):
    rng = np.random.default_rng(rows + width + columns)
    x, w, s, b = make(rng, rows, width, columns, bias=True)
    got = host(oi.w8a16_linear(dev(x), dev(w), dev(s), dev(b)))
    ref = gpu_f64_reference(x, w, s, b)
    assert tolerance.rel_err(got, ref) <= tolerance.FP16_REL_TOL


@pytest.mark.parametrize("route", ["0", "1", "2"])
@pytest.mark.parametrize("rows,width,columns", [(5, 64, 33), (16, 4096, 4096), (13, 4112, 77),
                                                (33, 1552, 200), (48, 16384, 17), (64, 8960, 1536),
                                                (7, 16, 3), (40, 4096, 8200), (60, 2048, 8300),
                                                (48, 4112, 9000)])
def test_skinny_rows_on_both_routes(oracle, monkeypatch, route, rows, width, columns, knobs):
    # 5..64 activation rows: the default choice (route 0), the skinny MFMA
    # kernel (OMNI_W8A16_ROUTE=1) and the tiled MFMA GEMM (=2) against the
    # f64 ground truth, with K tails that are not a multiple of 64 and
    # ragged column counts; (40, 4096, 8200) and (60, 2048, 8300) take the
    # GEMM by default, (48, 4112, 9000) stays skinny by default (no ring
    # kernel runs K % 64 != 0, and the register-staged GEMM only pays above
    # 48 rows).
    knobs.set("OMNI_W8A16_ROUTE", route)
    rng = np.random.default_rng(rows * 3 + width + columns)
    x, w, s, b = make(rng, rows, width, columns, bias=columns % 2 == 1)
    got = host(oi.w8a16_linear(dev(x), dev(w), dev(s), None if b is None else dev(b)))
    ref = gpu_f64_reference(x, w, s, b)
    assert tolerance.rel_err(got, ref) <= tolerance.FP16_REL_TOL, (route, rows, width, columns)


@pytest.mark.parametrize("kernel", ["0", "1"])
@pytest.mark.parametrize("rows,width,columns", [(5, 64, 33), (8, 960, 70), (16, 4096, 4096),
                                                (13, 2048, 17), (16, 4096, 129), (11, 4032, 300),
                                                (7, 1024, 50), (14, 3072, 101), (16, 3136, 64)])
def test_skinny_lds_kernel_and_fallback(oracle, monkeypatch, kernel, rows, width, columns, knobs):
    # 5..16 rows with K % 64 == 0 and K <= 4096: the LDS-staged skinny kernel
    # (0; its K = 1024 / 2048 / 3072 / 4096 builds and the run-time-K one) and
    # w8a16_skinny_kernel (OMNI_W8A16_SKINNY=1), with idle waves (K < 1024),
    # ragged column counts and bias, against the f64 truth.
    knobs.set("OMNI_W8A16_SKINNY", kernel)
    rng = np.random.default_rng(rows * 5 + width + columns)
    x, w, s, b = make(rng, rows, width, columns, bias=True)
    got = host(oi.w8a16_linear(dev(x), dev(w), dev(s), dev(b)))
    ref = gpu_f64_reference(x, w, s, b)
    assert tolerance.rel_err(got, ref) <= tolerance.FP16_REL_TOL, (kernel, rows, width, columns)


@pytest.mark.parametrize("tile", ["1", "2", "4", "5", "6", "7", "8", "9", "10", "11", "12", "16", "17", "18",
                                  "19", "20", "21"])
@pytest.mark.parametrize("rows,width,columns", [(300, 512, 200), (1024, 1536, 1536), (257, 8960, 129),
                                                (197, 4096, 640), (65, 64, 33), (600, 4096, 700)])
def test_every_prefill_kernel(oracle, monkeypatch, tile, rows, width, columns, knobs):
    # OMNI_W8A16_TILE pins one prefill kernel: the tiled GEMMs (1, 2) and the
    # LDS-DMA ring GEMMs (4 = 256 x 128, 5 = 128 x 128, 6 = 256 x 256, 7 = 256 x 256
    # with the waves side by side, 8 = 64 x 128, 9 = 256 x 192, 10 = 128 x 128
    # two workgroups per CU, 11 / 12 = 64 x 128 two / three per CU, 16 / 17 /
    # 18 = 128 x 256 / 256 x 256 / 256 x 256 with eight waves, 19 = 128 x 320,
    # whose tile has more columns than the workgroup has threads, so each
    # thread stages two columns' scale and bias, 20 / 21 = 64 x 192 /
    # 128 x 192); ragged rows/columns, bias, against the f64 ground truth
    knobs.set("OMNI_W8A16_TILE", tile)
    rng = np.random.default_rng(rows + width + columns + int(tile))
    x, w, s, b = make(rng, rows, width, columns, bias=True)
    got = host(oi.w8a16_linear(dev(x), dev(w), dev(s), dev(b)))
    ref = gpu_f64_reference(x, w, s, b)
    assert tolerance.rel_err(got, ref) <= tolerance.FP16_REL_TOL, (tile, rows, width, columns)


def test_config5_small_vlm_layer(oracle):
    # BASELINE config 5, one layer: prefill M=1024 then a decode step M=1
    rng = np.random.default_rng(5)
    hidden, ffn = 1536, 8960
    for rows in (1024, 1):
        for width, columns in ((hidden, hidden), (hidden, 512), (hidden, ffn), (ffn, hidden)):
            x, w, s, _ = make(rng, rows, width, columns)
            got = host(oi.w8a16_linear(dev(x), dev(w), dev(s)))
            ref = gpu_f64_reference(x, w, s, None)
            assert tolerance.rel_err(got, ref) <= tolerance.FP16_REL_TOL, (rows, width, columns)


@pytest.mark.parametrize("tile", ["4", "5", "8", "9", "10", "11", "12", "16", "17", "18", "19", "20", "21"])
@pytest.mark.parametrize("splits", ["2", "3", "5", "8"])
@pytest.mark.parametrize("rows,width,columns,bias", [(1024, 8960, 1536, False), (300, 1536, 202, True),
                                                     (257, 448, 129, True), (65, 64, 33, False),
                                                     (130, 4096, 515, True)])
def test_split_k_every_ring_kernel(oracle, monkeypatch, tile, splits, rows, width, columns, bias, knobs):
    # OMNI_W8A16_SPLITS forces split K on a pinned ring kernel: units of
    # (tile, K range), f32 partial sums, an in-order reduction applying scale
    # and bias. K tile counts 140, 24, 7 (uneven splits, fewer than asked
    # when a split would be empty) and 1 (no split), ragged rows and
    # columns, columns % 4 != 0 (the reduction's scalar path).
    knobs.set("OMNI_W8A16_TILE", tile)
    knobs.set("OMNI_W8A16_SPLITS", splits)
    rng = np.random.default_rng(rows + width + columns + 10 * int(tile) + int(splits))
    x, w, s, b = make(rng, rows, width, columns, bias=bias)
    xd, wd, sd, bd = dev(x), dev(w), dev(s), None if b is None else dev(b)
    got = oi.w8a16_linear(xd, wd, sd, bd)
    again = oi.w8a16_linear(xd, wd, sd, bd)
    ref = gpu_f64_reference(x, w, s, b)
    assert tolerance.rel_err(host(got), ref) <= tolerance.FP16_REL_TOL, (tile, splits, rows, width, columns)
    assert torch.equal(got, again), "split K must be deterministic"


def test_split_k_workspace_contract(monkeypatch, knobs):
    # omni_w8a16_gemm_workspace_size reports splits * rows * columns floats
    # for a split shape and 0 otherwise; omni_w8a16_gemm_ws splits less with
    # a smaller workspace, not at all with none, and every result is within
    # the bar.
    from omni_int8 import _lib
    L = _lib.lib()
    knobs.set("OMNI_W8A16_TILE", "12")
    knobs.set("OMNI_W8A16_SPLITS", "4")
    rows, width, columns = 192, 2048, 256
    assert L.omni_w8a16_gemm_workspace_size(rows, columns, width) == 4 * rows * columns * 4
    assert L.omni_w8a16_gemm_workspace_size(64, columns, width) == 0  # skinny route
    assert L.omni_w8a16_gemm_workspace_size(4, columns, width) == 0  # GEMV
    knobs.unset("OMNI_W8A16_TILE")
    knobs.unset("OMNI_W8A16_SPLITS")
    # the launcher's own choice: config 5's down projection splits, its
    # K = 1536 linears do not
    assert L.omni_w8a16_gemm_workspace_size(1024, 1536, 8960) % (1024 * 1536 * 4) == 0
    assert L.omni_w8a16_gemm_workspace_size(1024, 1536, 8960) >= 2 * 1024 * 1536 * 4
    assert L.omni_w8a16_gemm_workspace_size(1024, 8960, 1536) == 0
    rng = np.random.default_rng(78)
    x, w, s, b = make(rng, 1024, 8960, 1536)
    xd, wd, sd = dev(x), dev(w), dev(s)
    ref = gpu_f64_reference(x, w, s, None)
    out = torch.empty((1024, 1536), dtype=torch.float16, device="cuda")
    st = L.omni_w8a16_gemm(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), None, 1024, 1536, 8960, out.data_ptr(),
                           torch.cuda.current_stream().cuda_stream)
    assert st == 0, _lib.last_error()
    assert tolerance.rel_err(host(out), ref) <= tolerance.FP16_REL_TOL  # no workspace: unsplit
    assert tolerance.rel_err(host(oi.w8a16_linear(xd, wd, sd)), ref) <= tolerance.FP16_REL_TOL  # split
    # the plan asks for four splits of 128 x 192 tiles there; with room for
    # three or two it takes 128 x 128 tiles split two ways instead
    assert L.omni_w8a16_gemm_workspace_size(1024, 1536, 8960) == 4 * 1024 * 1536 * 4
    for floats in (4 * 1024 * 1536, 3 * 1024 * 1536, 2 * 1024 * 1536):
        ws = torch.empty(floats * 4, dtype=torch.uint8, device="cuda")
        ws.fill_(0x5A)
        st = L.omni_w8a16_gemm_ws(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), None, 1024, 1536, 8960,
                                  out.data_ptr(), ws.data_ptr(), floats * 4, torch.cuda.current_stream().cuda_stream)
        assert st == 0, _lib.last_error()
        assert tolerance.rel_err(host(out), ref) <= tolerance.FP16_REL_TOL, floats
    knobs.set("OMNI_W8A16_TILE", "12")
    knobs.set("OMNI_W8A16_SPLITS", "4")
    rng = np.random.default_rng(77)
    x, w, s, b = make(rng, rows, width, columns, bias=True)
    xd, wd, sd, bd = dev(x), dev(w), dev(s), dev(b)
    ref = gpu_f64_reference(x, w, s, b)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for floats in (4 * rows * columns, 2 * rows * columns + 5, 0):
        ws = torch.empty(max(floats, 1) * 4, dtype=torch.uint8, device="cuda")
        out = torch.empty((rows, columns), dtype=torch.float16, device="cuda")
        st = L.omni_w8a16_gemm_ws(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), rows, columns,
                                  width, out.data_ptr(), ws.data_ptr() if floats else None, floats * 4, stream)
        assert st == 0, _lib.last_error()
        assert tolerance.rel_err(host(out), ref) <= tolerance.FP16_REL_TOL, floats
        outs.append(out)
    knobs.set("OMNI_W8A16_SPLITS", "1")
    plain = oi.w8a16_linear(xd, wd, sd, bd)
    assert torch.equal(outs[2], plain), "no workspace runs unsplit"
    bad = torch.empty(1024, dtype=torch.uint8, device="cuda")
    st = L.omni_w8a16_gemm_ws(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), rows, columns, width,
                              outs[0].data_ptr(), bad.data_ptr() + 4, 512, stream)
    assert st == _lib.OMNI_BAD_ARGUMENT


@pytest.mark.parametrize("splits", ["auto", "2", "4", "8"])
@pytest.mark.parametrize("rows,width,columns,bias", [(16, 4096, 4096, False), (9, 2048, 1000, True),
                                                     (5, 8192, 300, True), (12, 256, 70, False),
                                                     (16, 1024, 4099, True), (13, 12288, 128, False),
                                                     (16, 3584, 8300, True), (8, 1344, 600, False)])
def test_skinny_split_k(oracle, monkeypatch, splits, rows, width, columns, bias, knobs):
    # The decode-shaped split-K kernel (5..16 rows): units of 64 columns x
    # K / splits, f32 partial sums, then the in-order reduction. Splits that
    # do not divide K into multiples of 256 of at most 1024 fall back to the
    # unsplit kernels; ragged columns, bias, K from 256 to 12288.
    if splits != "auto":
        knobs.set("OMNI_W8A16_SKINNY_SPLIT", splits)
    rng = np.random.default_rng(rows * 7 + width + columns + (0 if splits == "auto" else int(splits)))
    x, w, s, b = make(rng, rows, width, columns, bias=bias)
    xd, wd, sd, bd = dev(x), dev(w), dev(s), None if b is None else dev(b)
    got = oi.w8a16_linear(xd, wd, sd, bd)
    again = oi.w8a16_linear(xd, wd, sd, bd)
    ref = gpu_f64_reference(x, w, s, b)
    assert tolerance.rel_err(host(got), ref) <= tolerance.FP16_REL_TOL, (splits, rows, width, columns)
    assert torch.equal(got, again)
    knobs.set("OMNI_W8A16_SKINNY_SPLIT", "0")
    plain = oi.w8a16_linear(xd, wd, sd, bd)
    assert tolerance.rel_err(host(plain), ref) <= tolerance.FP16_REL_TOL


def test_skinny_split_k_workspace_size():
    from omni_int8 import _lib
    L = _lib.lib()
    # split where the unsplit kernel needs more than one round of 16-column
    # workgroups (N > 16 x 256 CUs), K <= 4096
    assert L.omni_w8a16_gemm_workspace_size(16, 14336, 4096) == 4 * 16 * 14336 * 4
    assert L.omni_w8a16_gemm_workspace_size(16, 8192, 2048) == 2 * 16 * 8192 * 4
    assert L.omni_w8a16_gemm_workspace_size(16, 4096, 4096) == 0                   # config 1: one round
    assert L.omni_w8a16_gemm_workspace_size(16, 8192, 1024) == 0                   # K fits one unit
    assert L.omni_w8a16_gemm_workspace_size(16, 8192, 4160) == 0                   # K > 4096
    assert L.omni_w8a16_gemm_workspace_size(16, 18944, 3584) == 4 * 16 * 18944 * 4  # 896-element units
    assert L.omni_w8a16_gemm_workspace_size(16, 8192, 8192) == 0                   # K > 4096
    assert L.omni_w8a16_gemm_workspace_size(17, 4096, 4096) == 0                   # skinny, not split
    # 17 rows of a 58.7 M-weight matrix take the GEMM, split K (64 x 128 tiles)
    assert L.omni_w8a16_gemm_workspace_size(17, 14336, 4096) % (17 * 14336 * 4) == 0
    assert L.omni_w8a16_gemm_workspace_size(17, 14336, 4096) >= 2 * 17 * 14336 * 4


@pytest.mark.parametrize("seed", range(12))
def test_default_routing_random_shapes(oracle, seed):
    # The default kernel choice (GEMV, skinny, split skinny, the rings by the
    # rounds model with or without split K, or the tiled fallback) on random
    # shapes: rows 1..900, widths multiples of 16 up to 9000
    rng = np.random.default_rng(2000 + seed)
    rows = int(rng.choice([1, 2, 4, 5, 16, 17, 64, 65, 300, 900]))
    width = 16 * int(rng.integers(1, 560))
    columns = int(rng.integers(1, 1200))
    x, w, s, b = make(rng, rows, width, columns, bias=bool(seed % 2))
    got = host(oi.w8a16_linear(dev(x), dev(w), dev(s), None if b is None else dev(b)))
    ref = gpu_f64_reference(x, w, s, b)
    assert tolerance.rel_err(got, ref) <= tolerance.FP16_REL_TOL, (rows, width, columns)
