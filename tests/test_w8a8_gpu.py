"""W8A8 parity on the GPU: the HIP kernels against the CPU oracle (bit-exact).

Mirrors the reference's own tests — crates/omni-kernel/src/int8_matmul.rs:700-786
(hand value, 64^3 tile fixture, negative control, both lowerings) and
prototypes/int8-gemm/src/main.rs:69-89 (check shapes) — then covers the
BASELINE configs at full size. Integer accumulators and the f32 epilogue are
compared for exact equality; nothing here has a tolerance except where the
reference's own test has one.
"""
import numpy as np
import pytest
import torch

import omni_int8 as oi

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


def weights(rng, columns, width):
    return rng.integers(-127, 128, (columns, width), dtype=np.int8)


def run_gemm(x, w, scale, zero, lowering=oi.OMNI_LOWERING_AUTO, bias=None, out_dtype=torch.float32):
    codes, rs, total = oi.quantize_rows(dev(x))
    out, acc = oi.w8a8_gemm(codes, rs, total, dev(w), dev(scale), dev(zero),
                            bias=None if bias is None else dev(bias), out_dtype=out_dtype,
                            acc_dump=True, lowering=lowering)
    return host(codes), host(rs), host(total), host(out), host(acc)


# -- quantisation ----------------------------------------------------------------


@pytest.mark.parametrize("rows,width", [(1, 4), (3, 12), (17, 36), (5, 100), (9, 2048), (33, 2064),
                                        (40, 3072), (64, 4096), (7, 12288), (2, 4100)])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_quantize_rows_bit_exact(oracle, rows, width, dtype):
    rng = np.random.default_rng(rows * 1000 + width)
    x = rng.standard_normal((rows, width)).astype(dtype)
    if rows > 2:
        x[1] = 0  # zero row: the 1e-30 floor
    codes, rs, total = oi.quantize_rows(dev(x))
    ocodes, ors, ototal = oracle.quantize_rows(x.astype(np.float32))
    assert np.array_equal(host(codes), ocodes)
    assert np.array_equal(host(rs).view(np.uint32), ors.view(np.uint32))
    assert np.array_equal(host(total), ototal)


def test_quantize_rows_ties_and_strided_input(oracle):
    # peak 127 -> row_scale 1: exact half-way quotients, and the f32 add in
    # floor(|q| + 0.5) that sends 0.49999997 to 1 (int8_matmul.rs:106).
    row = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -126.5, 0.49999997, -0.49999997, 1.5,
                    -1.5, 0.0], np.float32)
    x = np.tile(row, (3, 1))
    big = np.zeros((3, 20), np.float32)
    big[:, :12] = x
    strided = dev(big)[:, :12]  # leading dimension 20
    codes, rs, total = oi.quantize_rows(strided)
    assert host(codes)[0].tolist() == [127, 3, -3, 1, -1, 127, -127, 1, -1, 2, -2, 0]
    ocodes, _, ototal = oracle.quantize_rows(x)
    assert np.array_equal(host(codes), ocodes) and np.array_equal(host(total), ototal)


def test_quantize_rows_near_ties_at_random_scales(oracle):
    # Quotients within a few ulps of k + 0.5 at row scales from 2^-107 to 2^33:
    # the division must be correctly rounded for every code to match.
    rng = np.random.default_rng(11)
    rows, width = 512, 256
    peaks = np.ldexp(1.0 + rng.random(rows), rng.integers(-100, 40, rows)).astype(np.float32)
    s = np.maximum(peaks / np.float32(127), np.float32(1e-30)).astype(np.float32)
    k = rng.integers(0, 127, (rows, width))
    h = ((k + 0.5) * s[:, None].astype(np.float64)).astype(np.float32)
    h = (h.view(np.int32) + rng.integers(-4, 5, (rows, width)).astype(np.int32)).view(np.float32)
    x = np.minimum(h, peaks[:, None]) * np.where(rng.random((rows, width)) < 0.5, -1, 1).astype(np.float32)
    x[:, 0] = peaks
    codes, rs, total = oi.quantize_rows(dev(x))
    ocodes, ors, ototal = oracle.quantize_rows(x)
    assert np.array_equal(host(rs).view(np.uint32), ors.view(np.uint32))
    assert np.array_equal(host(codes), ocodes)
    assert np.array_equal(host(total), ototal)


@pytest.mark.parametrize("width", [256, 3072, 4096, 12288, 20000])
def test_quantize_rows_nan_and_inf(oracle, width):
    # Rust's f32::max skips NaN in the peak, and a NaN code converts to 0
    # (int8_host.rs:3-10); an Inf peak makes every finite code 0.
    rng = np.random.default_rng(width)
    x = rng.standard_normal((6, width)).astype(np.float32)
    x[0, 3] = np.nan
    x[1, 5] = np.inf
    x[2, 7] = -np.inf
    x[3, :] = np.nan
    x[4, 1] = np.nan
    x[4, 2] = np.inf
    codes, rs, total = oi.quantize_rows(dev(x))
    ocodes, ors, ototal = oracle.quantize_rows(x)
    assert np.array_equal(host(codes), ocodes)
    assert np.array_equal(host(rs).view(np.uint32), ors.view(np.uint32))
    assert np.array_equal(host(total), ototal)


# -- the reference's own tests ------------------------------------------------------


@pytest.mark.parametrize("lowering", [oi.OMNI_LOWERING_AUTO, oi.OMNI_LOWERING_SCALAR])
def test_hand_value_and_tile64_fixture(oracle, lowering):
    # int8_matmul.rs:749-786: hand value on the scalar kernel, then the 64^3
    # tile fixture on both lowerings, with the got+1 negative control.
    x = np.array([[1.0, -2.0, 0.5, 4.0]], np.float32)
    w = np.array([[1, -2, 3, -4]], np.int8)
    scale, zero = np.array([0.25], np.float32), np.array([1], np.int32)
    expected = oracle.dequant_reference(x, w, scale, zero)
    assert abs(expected[0, 0] - (-411.0 / 127.0)) < 1e-5
    got = host(oi.try_int8_gemm(dev(x), dev(oracle.pack_i8(w)), dev(scale), dev(zero)))
    assert np.max(np.abs(got - expected)) < 1e-3
    assert abs(got[0, 0] + 1.0 - expected[0, 0]) >= 1e-3

    x = np.zeros((64, 64), np.float32)
    x[0, :4] = [1.0, -2.0, 0.5, 4.0]
    w = np.zeros((64, 64), np.int8)
    w[0, :4] = [1, -2, 3, -4]
    scale = np.full(64, 0.25, np.float32)
    zero = np.zeros(64, np.int32)
    zero[0] = 1
    expected = oracle.dequant_reference(x, w, scale, zero)
    *_, out, acc = run_gemm(x, w, scale, zero, lowering=lowering)
    assert np.max(np.abs(out - expected)) < 1e-3
    assert abs(out[0, 0] + 1.0 - expected[0, 0]) >= 1e-3
    assert np.array_equal(out, oracle.int8_gemm(x, w, scale, zero))


@pytest.mark.parametrize("rows,width,columns", [(5, 12, 6), (17, 36, 14)])
def test_prototype_check_shapes(oracle, rows, width, columns):
    # prototypes/int8-gemm/src/main.rs:69-89 (widths not a multiple of 16: scalar lowering)
    i = np.arange(rows * width)
    x = (((i * 17) % 41) - 20).astype(np.float32).reshape(rows, width)
    w = (((np.arange(columns * width) * 13) % 31) - 15).astype(np.int8).reshape(columns, width)
    scale = (0.05 + np.arange(columns, dtype=np.float32) * 0.01).astype(np.float32)
    zero = ((np.arange(columns) % 5) - 2).astype(np.int32)
    got = host(oi.try_int8_gemm(dev(x), dev(oracle.pack_i8(w)), dev(scale), dev(zero)))
    want = oracle.int8_gemm(x, w, scale, zero)
    assert np.max(np.abs(got - want)) < 1e-3       # the prototype's bar
    assert np.array_equal(got, want)               # and in fact bit-exact


def test_try_int8_gemm_returns_none_on_shape_mismatch():
    x = torch.zeros((2, 8), device="cuda")
    assert oi.try_int8_gemm(x, torch.zeros(3, dtype=torch.int32, device="cuda"),
                            torch.ones(2, device="cuda"), torch.zeros(2, dtype=torch.int32, device="cuda")) is None
    assert oi.try_int8_gemm(torch.zeros((2, 6), device="cuda"), torch.zeros(3, dtype=torch.int32, device="cuda"),
                            torch.ones(2, device="cuda"), torch.zeros(2, dtype=torch.int32, device="cuda")) is None


# -- both lowerings, ragged shapes, epilogue variants ------------------------------------


SHAPES = [(1, 16, 1), (1, 64, 7), (3, 48, 5), (64, 64, 64), (255, 208, 129), (257, 4112, 300),
          (300, 512, 513), (16, 1024, 2048)]


@pytest.mark.parametrize("rows,width,columns", SHAPES)
@pytest.mark.parametrize("lowering", [oi.OMNI_LOWERING_MFMA, oi.OMNI_LOWERING_SCALAR])
def test_w8a8_bit_exact_ragged(oracle, rows, width, columns, lowering):
    rng = np.random.default_rng(rows + 7 * width + 13 * columns)
    x = rng.standard_normal((rows, width)).astype(np.float32)
    w = rng.integers(-128, 128, (columns, width), dtype=np.int8)
    scale = rng.uniform(0.002, 0.02, columns).astype(np.float32)
    zero = rng.integers(-4, 5, columns).astype(np.int32)
    bias = rng.standard_normal(columns).astype(np.float32)
    codes, rs, total, out, acc = run_gemm(x, w, scale, zero, lowering=lowering)
    oacc = oracle.int8_acc(codes, w)
    assert np.array_equal(acc, oacc)
    o32, _ = oracle.w8a8_finish(oacc, total, rs, scale, zero)
    assert np.array_equal(out.view(np.uint32), o32.view(np.uint32))
    # fp16 output with bias: one RNE rounding of the f32 value + bias
    *_, out16, _ = run_gemm(x, w, scale, zero, lowering=lowering, bias=bias, out_dtype=torch.float16)
    _, o16 = oracle.w8a8_finish(oacc, total, rs, scale, zero, bias)
    assert np.array_equal(out16.view(np.uint16), o16)


def test_w8a8_extreme_codes_no_overflow(oracle):
    # |acc| = 128 * 128 * K at K = 16384 is 2^28: exact in int32
    width = 16384
    x = np.full((3, width), -1.0, np.float32)
    x[:, 0] = 1.0  # codes: -127 mostly
    w = np.full((40, width), -128, np.int8)
    scale = np.full(40, 0.01, np.float32)
    zero = np.zeros(40, np.int32)
    codes, rs, total, out, acc = run_gemm(x, w, scale, zero, lowering=oi.OMNI_LOWERING_MFMA)
    assert np.array_equal(acc, oracle.int8_acc(codes, w))


# Every MFMA kernel variant (OMNI_W8A8_TILE; 0 = the shape heuristic) on
# shapes with ragged M/N edges, K tails and multi-round tile grids.
VARIANT_SHAPES = [(300, 1024, 700), (1000, 4096, 1500), (513, 4160, 389), (700, 3072, 650),
                  (2048, 2048, 3072), (4400, 512, 4100)]
TILE_VARIANTS = [3, 4, 9, 10, 11, 12, 13, 14, 15, 16, 17, 19]  # OMNI_W8A8_TILE values


@pytest.mark.parametrize("tile", [0] + TILE_VARIANTS)
def test_w8a8_every_kernel_variant(oracle, tile, monkeypatch, knobs):
    knobs.set("OMNI_W8A8_TILE", str(tile))
    for rows, width, columns in VARIANT_SHAPES:
        rng = np.random.default_rng(tile * 100 + rows)
        x = rng.standard_normal((rows, width)).astype(np.float16)
        w = rng.integers(-128, 128, (columns, width), dtype=np.int8)
        scale = rng.uniform(0.002, 0.02, columns).astype(np.float32)
        zero = rng.integers(-3, 4, columns).astype(np.int32)
        codes, rs, total = oi.quantize_rows(dev(x))
        out, acc = oi.w8a8_gemm(codes, rs, total, dev(w), dev(scale), dev(zero), acc_dump=True,
                                lowering=oi.OMNI_LOWERING_MFMA)
        exact = codes.double() @ dev(w).double().T
        assert torch.equal(acc.double(), exact), (tile, rows, width, columns)
        ref = ((acc - total[:, None] * dev(zero)[None, :]).float() * rs[:, None]) * dev(scale)[None, :]
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), (tile, rows, width, columns)


@pytest.mark.parametrize("tile", [16, 17])
def test_w8a8_pair_ring_short_and_odd_k(oracle, tile, monkeypatch, knobs):
    # The pair-refill ring takes any K % 64 == 0: fewer K tiles than the ring
    # (1, 2, 3, 5), exactly one unrolled pass (10), one more (11), and odd
    # counts where a pair's second tile is clamped to the last one.
    knobs.set("OMNI_W8A8_TILE", str(tile))
    for rows, width, columns in [(300, 64, 700), (300, 128, 389), (513, 192, 700), (257, 320, 513),
                                 (1000, 640, 1500), (600, 704, 400), (520, 1344, 260)]:
        rng = np.random.default_rng(tile * 1000 + width)
        x = rng.standard_normal((rows, width)).astype(np.float16)
        w = rng.integers(-128, 128, (columns, width), dtype=np.int8)
        scale = rng.uniform(0.002, 0.02, columns).astype(np.float32)
        zero = rng.integers(-3, 4, columns).astype(np.int32)
        codes, rs, total = oi.quantize_rows(dev(x))
        out, acc = oi.w8a8_gemm(codes, rs, total, dev(w), dev(scale), dev(zero), acc_dump=True,
                                lowering=oi.OMNI_LOWERING_MFMA)
        exact = codes.double() @ dev(w).double().T
        assert torch.equal(acc.double(), exact), (tile, rows, width, columns)
        ref = ((acc - total[:, None] * dev(zero)[None, :]).float() * rs[:, None]) * dev(scale)[None, :]
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), (tile, rows, width, columns)
        plain = oi.w8a8_gemm(codes, rs, total, dev(w), dev(scale), dev(zero), lowering=oi.OMNI_LOWERING_MFMA)
        assert torch.equal(plain.view(torch.int32), out.view(torch.int32)), (tile, rows, width, columns)


def wrap_i32(t):
    """int64 tensor -> its value modulo 2^32 as a signed int32 tensor."""
    return (((t + 2**31) % 2**32) - 2**31).to(torch.int32)


@pytest.mark.parametrize("tile", [0] + TILE_VARIANTS)
def test_w8a8_wide_row_sums_and_zero_points(oracle, tile, monkeypatch, knobs):
    # The epilogue forms acc - row_sum * zero in 24-bit multiplies while every
    # row sum and zero point of a tile lies in [-2^23, 2^23), and in 32-bit
    # ones otherwise: caller-supplied sums and zero points at, inside and
    # outside that range (one wide row or column is enough to switch a whole
    # tile), with the product wrapping modulo 2^32 as int32 arithmetic does.
    knobs.set("OMNI_W8A8_TILE", str(tile))
    rows, width, columns = 600, 1024, 520
    rng = np.random.default_rng(400 + tile)
    codes = dev(rng.integers(-127, 128, (rows, width), dtype=np.int8))
    w = dev(rng.integers(-128, 128, (columns, width), dtype=np.int8))
    rs = dev(rng.uniform(1e-4, 1e-2, rows).astype(np.float32))
    scale = dev(rng.uniform(0.002, 0.02, columns).astype(np.float32))
    edge = np.array([2**23 - 1, -2**23, 2**23, -2**23 - 1, 2**31 - 1, -2**31], np.int64)
    cases = []
    small_sum = rng.integers(-2**22, 2**22, rows)
    small_zero = rng.integers(-2**22, 2**22, columns)
    s1 = small_sum.copy(); s1[:2] = edge[:2]  # boundary values that still fit
    z1 = small_zero.copy(); z1[:2] = edge[:2]
    cases.append((s1, z1))
    s2 = small_sum.copy(); s2[300] = 2**23  # one wide row in the second M tile
    cases.append((s2, small_zero))
    z3 = small_zero.copy(); z3[517] = -2**23 - 1  # one wide column in the last N tile
    cases.append((small_sum, z3))
    cases.append((rng.integers(-2**31, 2**31, rows), rng.integers(-2**31, 2**31, columns)))
    acc = (codes.double() @ w.double().T).to(torch.int64)
    for sums, zeros in cases:
        total = dev(sums.astype(np.int32))
        zero = dev(zeros.astype(np.int32))
        out = oi.w8a8_gemm(codes, rs, total, w, scale, zero, lowering=oi.OMNI_LOWERING_MFMA)
        centered = wrap_i32(acc - total.long()[:, None] * zero.long()[None, :])
        ref = (centered.float() * rs[:, None]) * scale[None, :]
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), (tile, int(np.abs(sums).max()))


@pytest.mark.parametrize("tile", TILE_VARIANTS)
def test_w8a8_every_kernel_variant_f16_bias(oracle, tile, monkeypatch, knobs):
    # The f16-output and bias epilogue of each variant, on a ragged shape.
    knobs.set("OMNI_W8A8_TILE", str(tile))
    rows, width, columns = 700, 3072, 650
    rng = np.random.default_rng(tile)
    x = rng.standard_normal((rows, width)).astype(np.float16)
    w = rng.integers(-128, 128, (columns, width), dtype=np.int8)
    scale = rng.uniform(0.002, 0.02, columns).astype(np.float32)
    zero = rng.integers(-3, 4, columns).astype(np.int32)
    bias = rng.standard_normal(columns).astype(np.float32)
    codes, rs, total = oi.quantize_rows(dev(x))
    out = oi.w8a8_gemm(codes, rs, total, dev(w), dev(scale), dev(zero), bias=dev(bias),
                       out_dtype=torch.float16, lowering=oi.OMNI_LOWERING_MFMA)
    o32, o16 = oracle.w8a8_finish(oracle.int8_acc(host(codes), w), host(total), host(rs), scale, zero,
                                  bias)
    assert np.array_equal(host(out).view(np.uint16), o16), tile
    # f32 output with bias, and with all-zero zero points (the epilogue drops
    # the row-sum term for such tiles)
    out32 = oi.w8a8_gemm(codes, rs, total, dev(w), dev(scale), dev(zero), bias=dev(bias),
                         lowering=oi.OMNI_LOWERING_MFMA)
    assert np.array_equal(host(out32).view(np.uint32), o32.view(np.uint32)), tile
    z0 = np.zeros(columns, np.int32)
    out32z = oi.w8a8_gemm(codes, rs, total, dev(w), dev(scale), dev(z0), bias=dev(bias),
                          lowering=oi.OMNI_LOWERING_MFMA)
    o32z, _ = oracle.w8a8_finish(oracle.int8_acc(host(codes), w), host(total), host(rs), scale, z0, bias)
    assert np.array_equal(host(out32z).view(np.uint32), o32z.view(np.uint32)), tile


# -- BASELINE configs at full size ---------------------------------------------------


def exact_acc(codes, wd):
    """int32 accumulators of codes @ wd^T through an f64 GEMM on the GPU:
    every product and partial sum is an integer below 2^53, so f64 is exact."""
    return (codes.double() @ wd.double().T)


def full_size_check(oracle, rows, width, columns, seed, outliers=False, sample_rows=12):
    """Full-size check: the int32 accumulators against an exact f64 GEMM on the
    GPU, the f32 epilogue against the reference op order in torch f32, and
    sampled rows against the C oracle. The production build of the kernels
    (no accumulator dump: the instantiation the bench times) must give the
    same output bit for bit as the dumping build that is checked."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, width)).astype(np.float16)
    if outliers:  # 1% of channels x20 (diffusion config)
        ch = rng.choice(width, size=max(1, width // 100), replace=False)
        x[:, ch] = (x[:, ch].astype(np.float32) * 20).astype(np.float16)
    w = rng.integers(-127, 128, (columns, width), dtype=np.int8)
    scale = rng.uniform(0.002, 0.02, columns).astype(np.float32)
    zero = np.zeros(columns, np.int32)
    zero[::7] = 3  # a nonzero-zero-point parity case on every 7th channel
    xd, wd = dev(x), dev(w)
    codes, rs, total = oi.quantize_rows(xd)
    out, acc = oi.w8a8_gemm(codes, rs, total, wd, dev(scale), dev(zero), acc_dump=True)
    assert torch.equal(acc.double(), exact_acc(codes, wd))
    centered = acc - total[:, None] * dev(zero)[None, :]
    ref = (centered.float() * rs[:, None]) * dev(scale)[None, :]
    assert torch.equal(out.view(torch.int32), ref.view(torch.int32))
    del acc, centered
    plain = oi.w8a8_gemm(codes, rs, total, wd, dev(scale), dev(zero))
    assert torch.equal(plain.view(torch.int32), out.view(torch.int32))
    del plain
    # sampled rows through the C oracle from the f16 input (quantisation included)
    idx = np.unique(np.concatenate([[0, rows - 1], rng.choice(rows, sample_rows, replace=False)]))
    want = oracle.int8_gemm(x[idx].astype(np.float32), w, scale, zero)
    got = host(out)[idx]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("columns", [4096, 14336])
def test_config3_prefill_full_size(oracle, columns):
    # M = 4 x 512, K = 4096
    full_size_check(oracle, 2048, 4096, columns, seed=columns)


@pytest.mark.parametrize("columns", [4096, 14336])
def test_config3_f16_bias_epilogue_full_size(oracle, columns):
    # BASELINE config 3 as the bench runs it: zero points absent (w_zero and
    # row sums NULL), f32 bias, f16 output; every output against the oracle's
    # epilogue (int8_matmul.rs:156-158 plus the bias add and one RNE cast)
    # applied to the exact accumulators.
    rows, width = 2048, 4096
    rng = np.random.default_rng(31 + columns)
    x = rng.standard_normal((rows, width)).astype(np.float16)
    w = rng.integers(-127, 128, (columns, width), dtype=np.int8)
    scale = rng.uniform(0.002, 0.02, columns).astype(np.float32)
    bias = rng.standard_normal(columns).astype(np.float32)
    wd = dev(w)
    codes, rs, total = oi.quantize_rows(dev(x))
    out = oi.w8a8_gemm(codes, rs, None, wd, dev(scale), None, dev(bias), torch.float16)
    acc = exact_acc(codes, wd).to(torch.int32)
    _, o16 = oracle.w8a8_finish(host(acc), np.zeros(rows, np.int32), host(rs), scale,
                                np.zeros(columns, np.int32), bias)
    assert np.array_equal(host(out).view(np.uint16), o16)


@pytest.mark.parametrize("width,columns", [(3072, 9216), (3072, 12288), (12288, 3072)])
def test_config4_diffusion_full_size(oracle, width, columns):
    # M = 4096 + 256 tokens, 1% outlier channels x20
    full_size_check(oracle, 4352, width, columns, seed=width + columns, outliers=True, sample_rows=6)


@pytest.mark.parametrize("width,columns", [(3072, 12288), (12288, 3072)])
def test_north_star_gemm_full_size(oracle, width, columns):
    full_size_check(oracle, 4096, width, columns, seed=7, sample_rows=6)


@pytest.mark.parametrize("width,columns", [(3072, 12288), (12288, 3072)])
def test_north_star_try_int8_gemm_as_benched(oracle, width, columns):
    # The exact call the bench times: try_int8_gemm on f16 activations with
    # all-zero zero points, f32 out. Every output against the reference op
    # order applied to exact accumulators (of the codes the quantiser made,
    # which the oracle pins below), and sampled rows end to end (quantisation
    # included) against the C oracle.
    rows = 4096
    rng = np.random.default_rng(width ^ columns)
    x = rng.standard_normal((rows, width)).astype(np.float16)
    w = rng.integers(-127, 128, (columns, width), dtype=np.int8)
    scale = rng.uniform(0.002, 0.02, columns).astype(np.float32)
    zero = np.zeros(columns, np.int32)
    xd, wd = dev(x), dev(w)
    out = oi.try_int8_gemm(xd, wd.view(torch.int32).reshape(-1), dev(scale), dev(zero))
    codes, rs, total = oi.quantize_rows(xd)
    ref = (exact_acc(codes, wd).to(torch.int32).float() * rs[:, None]) * dev(scale)[None, :]
    assert torch.equal(out.view(torch.int32), ref.view(torch.int32))
    idx = np.unique(np.concatenate([[0, rows - 1], rng.choice(rows, 6, replace=False)]))
    ocodes, _, _ = oracle.quantize_rows(x[idx].astype(np.float32))
    assert np.array_equal(host(codes)[idx], ocodes)
    want = oracle.int8_gemm(x[idx].astype(np.float32), w, scale, zero)
    assert np.array_equal(host(out)[idx].view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("columns,width", [(4096, 4096), (12288, 4096), (4096, 12288)])
def test_try_int8_gemm_split_k_reference_shapes(oracle, columns, width):
    # The reference's own 256-row int8 GEMM benchmark shapes
    # (docs/qwen-image-convrot-optimization-research.md:5) through the
    # operator. With omni_try_int8_gemm_split_workspace_size bytes the GEMM
    # splits K where that pays (256 x 4096 from K = 4096 on; 256 x 12288 has
    # 96 tiles and does not split), with a workspace handed over full of
    # garbage: every output bit equal to the unsplit operator's (the plain
    # workspace), to a second call on the same workspace, to the no-alloc
    # entry (whose static scratch holds the split too), and to the C oracle
    # on sampled rows, with zero points.
    from omni_int8 import _lib
    L = _lib.lib()
    rows = 256
    rng = np.random.default_rng(columns + 7 * width)
    x = rng.standard_normal((rows, width)).astype(np.float16)
    w = rng.integers(-127, 128, (columns, width), dtype=np.int8)
    scale = rng.uniform(0.002, 0.02, columns).astype(np.float32)
    zero = rng.integers(-3, 4, columns).astype(np.int32)
    xd, wp, sd, zd = dev(x), dev(w).view(torch.int32).reshape(-1), dev(scale), dev(zero)
    plain_bytes = L.omni_try_int8_gemm_workspace_size(rows, width)
    split_bytes = L.omni_try_int8_gemm_split_workspace_size(rows, columns, width)
    assert (split_bytes > plain_bytes) == (columns == 4096), (plain_bytes, split_bytes)
    stream = torch.cuda.current_stream().cuda_stream

    def call(ws, nbytes):
        out = torch.empty((rows, columns), dtype=torch.float32, device="cuda")
        st = L.omni_try_int8_gemm(xd.data_ptr(), oi.OMNI_F16, rows, width, wp.data_ptr(), wp.numel(),
                                  sd.data_ptr(), columns, zd.data_ptr(), columns, out.data_ptr(),
                                  ws.data_ptr(), nbytes, stream)
        assert st == 0, _lib.last_error()
        return out

    plain = call(torch.empty(plain_bytes, dtype=torch.uint8, device="cuda"), plain_bytes)
    ws = torch.full((split_bytes,), 0x5A, dtype=torch.uint8, device="cuda")
    split = call(ws, split_bytes)
    again = call(ws, split_bytes)
    noalloc = torch.empty((rows, columns), dtype=torch.float32, device="cuda")
    st = L.omni_try_int8_gemm_noalloc(xd.data_ptr(), oi.OMNI_F16, rows, width, wp.data_ptr(), wp.numel(),
                                      sd.data_ptr(), columns, zd.data_ptr(), columns, noalloc.data_ptr(), stream)
    assert st == 0, _lib.last_error()
    for got in (split, again, noalloc, oi.try_int8_gemm(xd, wp, sd, zd)):
        assert torch.equal(got.view(torch.int32), plain.view(torch.int32))
    idx = np.array([0, 1, 77, 128, 200, rows - 1])
    want = oracle.int8_gemm(x[idx].astype(np.float32), w, scale, zero)
    assert np.array_equal(host(split)[idx].view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows,width,columns", [(1, 64, 7), (300, 512, 513), (700, 3072, 650),
                                                (1000, 4096, 1500)])
@pytest.mark.parametrize("lowering", [oi.OMNI_LOWERING_MFMA, oi.OMNI_LOWERING_SCALAR])
def test_w8a8_without_zero_points(oracle, rows, width, columns, lowering):
    # w_zero and x_sum NULL (the has_zero = false epilogue), f32 and f16+bias.
    rng = np.random.default_rng(rows * 3 + columns)
    x = rng.standard_normal((rows, width)).astype(np.float16)
    w = rng.integers(-128, 128, (columns, width), dtype=np.int8)
    scale = rng.uniform(0.002, 0.02, columns).astype(np.float32)
    bias = rng.standard_normal(columns).astype(np.float32)
    codes, rs, total = oi.quantize_rows(dev(x))
    out = oi.w8a8_gemm(codes, rs, None, dev(w), dev(scale), None, lowering=lowering)
    out16 = oi.w8a8_gemm(codes, rs, None, dev(w), dev(scale), None, dev(bias), torch.float16,
                         lowering=lowering)
    out32b = oi.w8a8_gemm(codes, rs, None, dev(w), dev(scale), None, dev(bias), lowering=lowering)
    oacc = oracle.int8_acc(host(codes), w)
    nz, cz = np.zeros(rows, np.int32), np.zeros(columns, np.int32)
    o32, _ = oracle.w8a8_finish(oacc, nz, host(rs), scale, cz)
    o32b, o16 = oracle.w8a8_finish(oacc, nz, host(rs), scale, cz, bias)
    assert np.array_equal(host(out).view(np.uint32), o32.view(np.uint32))
    assert np.array_equal(host(out16).view(np.uint16), o16)
    assert np.array_equal(host(out32b).view(np.uint32), o32b.view(np.uint32))


def test_w8a8_strided_scales_and_bias(oracle):
    # 1-D operands given as strided views: the host layer copies them
    # contiguous and keeps each copy alive until the call has returned, so no
    # two operands can share a recycled block.
    rows, width, columns = 300, 1024, 700
    rng = np.random.default_rng(5)
    x = rng.standard_normal((rows, width)).astype(np.float16)
    w = rng.integers(-128, 128, (columns, width), dtype=np.int8)
    scale = rng.uniform(0.002, 0.02, columns).astype(np.float32)
    zero = rng.integers(-3, 4, columns).astype(np.int32)
    bias = rng.standard_normal(columns).astype(np.float32)
    codes, rs, total = oi.quantize_rows(dev(x))

    def strided(a):
        t = torch.zeros((a.shape[0], 3), dtype=torch.from_numpy(a).dtype, device="cuda")
        t[:, 1] = dev(a)
        return t[:, 1]

    rs2 = torch.zeros((rows, 2), device="cuda")
    rs2[:, 0] = rs
    tot2 = torch.zeros((rows, 2), dtype=torch.int32, device="cuda")
    tot2[:, 0] = total
    s_v, z_v, b_v = strided(scale), strided(zero), strided(bias)
    assert not s_v.is_contiguous() and not b_v.is_contiguous()
    for _ in range(3):
        out = oi.w8a8_gemm(codes, rs2[:, 0], tot2[:, 0], dev(w), s_v, z_v, b_v, torch.float16)
        oacc = oracle.int8_acc(host(codes), w)
        _, o16 = oracle.w8a8_finish(oacc, host(total), host(rs), scale, zero, bias)
        assert np.array_equal(host(out).view(np.uint16), o16)


def test_w8a8_rejects_bad_vectors():
    codes = torch.zeros((4, 64), dtype=torch.int8, device="cuda")
    w = torch.zeros((8, 64), dtype=torch.int8, device="cuda")
    rs = torch.ones(4, device="cuda")
    s = torch.ones(8, device="cuda")
    z = torch.zeros(8, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError):  # row sums of the wrong dtype
        oi.w8a8_gemm(codes, rs, torch.zeros(4, device="cuda"), w, s, z)
    with pytest.raises(ValueError):  # row sums of the wrong length
        oi.w8a8_gemm(codes, rs, torch.zeros(3, dtype=torch.int32, device="cuda"), w, s, z)
    with pytest.raises(ValueError):  # zero points without row sums
        oi.w8a8_gemm(codes, rs, None, w, s, z)


@pytest.mark.parametrize("splits", [2, 3, 4, 8])
def test_w8a8_split_k_bit_identical(oracle, splits, monkeypatch, knobs):
    # OMNI_W8A8_SPLITS forces split K on the 256 x 128 pair ring: int32
    # partial sums of (tile, K range) units, then a reduction applying the
    # epilogue. Every output (f32 and f16, bias, zero points or none, wide
    # row sums and zero points) and the accumulators must equal the unsplit
    # kernel's bit for bit; K tile counts 64, 24, 7 (uneven splits, fewer
    # than asked when a split would be empty) and 1 (no split), ragged rows
    # and columns, columns % 4 != 0 (the reduction's scalar path).
    knobs.set("OMNI_W8A8_TILE", "17")
    for rows, width, columns in [(256, 4096, 4096), (300, 1536, 202), (513, 448, 129), (70, 64, 33),
                                 (257, 4096, 515)]:
        rng = np.random.default_rng(splits * 1000 + width + columns)
        codes = dev(rng.integers(-128, 128, (rows, width), dtype=np.int8))
        w = dev(rng.integers(-128, 128, (columns, width), dtype=np.int8))
        rs = dev(rng.uniform(1e-4, 1e-2, rows).astype(np.float32))
        scale = dev(rng.uniform(0.002, 0.02, columns).astype(np.float32))
        bias = dev(rng.standard_normal(columns).astype(np.float32))
        small = (dev(rng.integers(-5000, 5000, rows).astype(np.int32)),
                 dev(rng.integers(-3, 4, columns).astype(np.int32)))
        wide = (dev(rng.integers(-2**31, 2**31, rows).astype(np.int32)),
                dev(rng.integers(-2**31, 2**31, columns).astype(np.int32)))
        for total, zero in (small, wide, (None, None)):
            for b in (None, bias):
                for odt in (torch.float32, torch.float16):
                    knobs.unset("OMNI_W8A8_SPLITS")
                    ref, ref_acc = oi.w8a8_gemm(codes, rs, total, w, scale, zero, bias=b, out_dtype=odt,
                                                acc_dump=True, lowering=oi.OMNI_LOWERING_MFMA)
                    knobs.set("OMNI_W8A8_SPLITS", str(splits))
                    got, acc = oi.w8a8_gemm(codes, rs, total, w, scale, zero, bias=b, out_dtype=odt,
                                            acc_dump=True, lowering=oi.OMNI_LOWERING_MFMA)
                    plain = oi.w8a8_gemm(codes, rs, total, w, scale, zero, bias=b, out_dtype=odt,
                                         lowering=oi.OMNI_LOWERING_MFMA)
                    case = (splits, rows, width, columns, total is None, b is None, odt)
                    assert torch.equal(acc, ref_acc), case
                    assert torch.equal(got.view(torch.int8), ref.view(torch.int8)), case
                    assert torch.equal(plain.view(torch.int8), ref.view(torch.int8)), case
        exact = codes.double() @ w.double().T
        assert torch.equal(ref_acc.double(), exact)


def test_w8a8_split_k_workspace_contract(monkeypatch):
    # omni_w8a8_gemm_workspace_size: the reference's 256-row benchmark shapes
    # with 32 tiles split, 256 x 12288 x 4096 (96 tiles) and the north-star
    # shapes do not; omni_w8a8_gemm_ws splits less with a smaller workspace
    # and not at all with none, bit-identically.
    from omni_int8 import _lib
    L = _lib.lib()
    for m, n, k in ((256, 4096, 12288), (256, 4096, 4096)):
        size = L.omni_w8a8_gemm_workspace_size(m, n, k)
        assert size >= 2 * m * n * 4 and size % (m * n * 4) == 0, (m, n, k, size)
    for m, n, k in ((256, 12288, 4096), (512, 4096, 4096), (4096, 12288, 3072), (4096, 3072, 12288)):
        assert L.omni_w8a8_gemm_workspace_size(m, n, k) == 0, (m, n, k)
    rows, width, columns = 256, 8192, 1024
    rng = np.random.default_rng(91)
    codes = dev(rng.integers(-128, 128, (rows, width), dtype=np.int8))
    w = dev(rng.integers(-128, 128, (columns, width), dtype=np.int8))
    rs = dev(rng.uniform(1e-4, 1e-2, rows).astype(np.float32))
    scale = dev(rng.uniform(0.002, 0.02, columns).astype(np.float32))
    total = dev(rng.integers(-5000, 5000, rows).astype(np.int32))
    zero = dev(rng.integers(-3, 4, columns).astype(np.int32))
    ref = oi.w8a8_gemm(codes, rs, total, w, scale, zero)
    stream = torch.cuda.current_stream().cuda_stream
    for nbytes in (4 * rows * columns * 4, (2 * rows * columns + 3) * 4, 0):
        ws = torch.full((max(nbytes, 1),), 0x5A, dtype=torch.uint8, device="cuda")
        for call in range(2):  # the same workspace again: it needs no initialisation
            out = torch.empty((rows, columns), dtype=torch.float32, device="cuda")
            st = L.omni_w8a8_gemm_ws(codes.data_ptr(), rs.data_ptr(), total.data_ptr(), w.data_ptr(),
                                     scale.data_ptr(), zero.data_ptr(), None, rows, columns, width,
                                     out.data_ptr(), oi.OMNI_F32, None, oi.OMNI_LOWERING_AUTO,
                                     ws.data_ptr() if nbytes else None, nbytes, stream)
            assert st == 0, _lib.last_error()
            assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), (nbytes, call)
    bad = torch.empty(1024, dtype=torch.uint8, device="cuda")
    st = L.omni_w8a8_gemm_ws(codes.data_ptr(), rs.data_ptr(), total.data_ptr(), w.data_ptr(), scale.data_ptr(),
                             zero.data_ptr(), None, rows, columns, width, out.data_ptr(), oi.OMNI_F32, None,
                             oi.OMNI_LOWERING_AUTO, bad.data_ptr() + 4, 512, stream)
    assert st == _lib.OMNI_BAD_ARGUMENT
