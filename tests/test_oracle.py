"""Pins for the CPU oracle (CPU only).

Each test checks one oracle function against something other than its own
formula: the reference's hand values and fixtures (file:line cited), numpy as
an independent implementation of IEEE conversions and exact integer products,
and mathematical invariants. Every test plants nothing in the product.
"""
import numpy as np
import pytest

import tolerance

# -- fp16 conversions ---------------------------------------------------------


def test_f16_to_f32_all_halves_match_numpy(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne(oracle):
    rng = np.random.default_rng(0)
    pats = rng.integers(0, 2**32, size=1 << 17, dtype=np.uint64).astype(np.uint32)
    vals = pats.view(np.float32)
    specials = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e-8, 2.0**-24,
                         2.0**-25, 2.0**-25 * 1.0000001, 3 * 2.0**-26, 2.0**-14, 2.0**-14 * 0.999,
                         1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, np.inf, -np.inf, 1e30, -1e-30],
                        dtype=np.float32)
    # halves' midpoints: exact ties in both directions
    h = np.arange(0, 0x7C00, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    vals = np.concatenate([vals, specials, mids, -mids])
    got = oracle.f32_to_f16_bits(vals)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got.view(np.float16)), nan)
    assert np.array_equal(got[~nan], want[~nan].view(np.uint16))


# -- round_half_away / packing (int8_host.rs:3-17, convrot.rs:151-160) --------


@pytest.mark.parametrize("value,code", [
    (0.5, 1), (-0.5, -1), (1.5, 2), (-1.5, -2), (2.5, 3), (-2.5, -3),
    # the reference adds 0.5 in f32 before floor: 0.49999997 + 0.5 rounds to 1.0
    (0.49999997, 1), (-0.49999997, -1), (0.4999999, 0), (126.5, 127), (127.5, 127), (-127.5, -128), (-128.5, -128),
    (1000.0, 127), (-1000.0, -128), (0.0, 0), (-0.0, 0), (float("nan"), 0),
])
def test_round_half_away_ties_and_clamp(oracle, value, code):
    assert oracle.round_half_away(value) == code


def test_pack_unpack_every_byte(oracle):
    codes = np.arange(-128, 128, dtype=np.int8)
    words = oracle.pack_i8(codes)
    assert np.array_equal(words.view(np.int8), codes)  # byte identity, little endian
    assert words[0] == int.from_bytes(bytes([0x80, 0x81, 0x82, 0x83]), "little", signed=True)
    assert np.array_equal(oracle.unpack_i8(words), codes)


# -- quantize_rows (int8_matmul.rs:23-118, int8_host.rs:31-39) -----------------


def test_quantize_hand_codes(oracle):
    # int8_matmul.rs:757: codes 32, -64, 16, 127 for x = [1, -2, 0.5, 4].
    codes, scale, total = oracle.quantize_rows(np.array([[1.0, -2.0, 0.5, 4.0]], np.float32))
    assert codes.tolist() == [[32, -64, 16, 127]]
    assert scale[0] == np.float32(4.0) / np.float32(127.0)
    assert total[0] == 111


def test_quantize_exact_halfway_inputs_round_away(oracle):
    # peak 127 -> row_scale exactly 1, so x / row_scale is exact.
    x = np.array([[127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -126.5, 3.49999976, -127.0, 0.0, 1.5, -1.5]],
                 np.float32)
    codes, scale, total = oracle.quantize_rows(x)
    assert scale[0] == 1.0
    assert codes[0].tolist() == [127, 3, -3, 1, -1, 127, -127, 3, -127, 0, 2, -2]
    assert total[0] == int(codes[0].astype(np.int64).sum())


def test_quantize_zero_row_uses_floor(oracle):
    codes, scale, total = oracle.quantize_rows(np.zeros((2, 8), np.float32))
    assert np.all(codes == 0) and np.all(total == 0)
    assert np.all(scale == np.float32(1e-30))


def test_quantize_random_rows_bounds_and_numpy(oracle):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 1024)).astype(np.float32)
    x[3] *= 1e-20  # tiny row
    x[5, 7] = 50.0  # outlier
    codes, scale, total = oracle.quantize_rows(x)
    peak = np.abs(x).max(axis=1)
    # every nonzero row reaches +-127 at its peak, and |code*scale - x| <= scale/2
    assert np.all(np.abs(codes).max(axis=1) == 127)
    err = np.abs(codes.astype(np.float64) * scale[:, None] - x)
    assert np.all(err <= scale[:, None].astype(np.float64) * (0.5 + 1e-5))
    assert np.array_equal(total, codes.astype(np.int64).sum(axis=1))
    # numpy float32 restatement (independent rounding primitives)
    s = np.maximum(peak / np.float32(127), np.float32(1e-30)).astype(np.float32)
    q = x / s[:, None]
    r = np.where(q >= 0, np.floor(q + np.float32(0.5)), np.ceil(q - np.float32(0.5)))
    assert np.array_equal(codes, np.clip(r, -128, 127).astype(np.int8))
    assert np.array_equal(scale, s)


# -- integer core and epilogue (int8_host.rs:19-53) -----------------------------


def test_int8_acc_matches_exact_integer_product(oracle):
    rng = np.random.default_rng(2)
    a = rng.integers(-128, 128, (33, 260), dtype=np.int8)
    w = rng.integers(-128, 128, (45, 260), dtype=np.int8)
    assert np.array_equal(oracle.int8_acc(a, w), a.astype(np.int64) @ w.astype(np.int64).T)
    # extreme codes: |acc| = 128*128*K fits int32 for the shapes here
    a = np.full((2, 4096), -128, np.int8)
    w = np.full((3, 4096), -128, np.int8)
    assert np.all(oracle.int8_acc(a, w) == 128 * 128 * 4096)


def _hand():
    x = np.array([[1.0, -2.0, 0.5, 4.0]], np.float32)
    w = np.array([[1, -2, 3, -4]], np.int8)
    return x, w, np.array([0.25], np.float32), np.array([1], np.int32)


def test_hand_value_matches_reference(oracle):
    # int8_matmul.rs:700-732: acc -300, sum 111, centered -411 -> -411/127.
    x, w, scale, zero = _hand()
    codes, _, _ = oracle.quantize_rows(x)
    assert oracle.int8_acc(codes, w)[0, 0] == -300
    got = oracle.int8_gemm(x, w, scale, zero)
    expected = oracle.dequant_reference(x, w, scale, zero)
    assert abs(expected[0, 0] - (-411.0 / 127.0)) < 1e-4          # :709
    assert abs(got[0, 0] - expected[0, 0]) < 1e-3                  # :731
    assert abs(got[0, 0] + 1.0 - expected[0, 0]) >= 1e-3           # negative control :768


@pytest.mark.parametrize("rows,width,columns", [(5, 12, 6), (17, 36, 14)])
def test_prototype_check_shapes(oracle, rows, width, columns):
    # prototypes/int8-gemm/src/main.rs:69-89
    i = np.arange(rows * width)
    x = (((i * 17) % 41) - 20).astype(np.float32).reshape(rows, width)
    w = (((np.arange(columns * width) * 13) % 31) - 15).astype(np.int8).reshape(columns, width)
    scale = (0.05 + np.arange(columns, dtype=np.float32) * 0.01).astype(np.float32)
    zero = ((np.arange(columns) % 5) - 2).astype(np.int32)
    got = oracle.int8_gemm(x, w, scale, zero)
    # the integer reference recomputed with numpy integers + the f32 epilogue
    codes, rs, total = oracle.quantize_rows(x)
    acc = codes.astype(np.int64) @ w.astype(np.int64).T
    centered = (acc - total[:, None].astype(np.int64) * zero[None, :]).astype(np.float32)
    want = (centered * rs[:, None]) * scale[None, :]
    # main.rs:79-85 holds the kernels to 1e-3 of this integer reference; the
    # restatement must meet it exactly.
    assert np.array_equal(got, want.astype(np.float32))


def test_tile64_fixture(oracle):
    # int8_matmul.rs:734-747: 64x64x64, one live row/column, zero[0] = 1.
    x = np.zeros((64, 64), np.float32)
    x[0, :4] = [1.0, -2.0, 0.5, 4.0]
    w = np.zeros((64, 64), np.int8)
    w[0, :4] = [1, -2, 3, -4]
    scale = np.full(64, 0.25, np.float32)
    zero = np.zeros(64, np.int32)
    zero[0] = 1
    expected = oracle.dequant_reference(x, w, scale, zero)
    assert abs(expected[0, 0] - (-411.0 / 127.0)) < 1e-5
    got = oracle.int8_gemm(x, w, scale, zero)
    assert np.max(np.abs(got - expected)) < 1e-3
    want = np.zeros((64, 64), np.float32)
    want[0, 0] = got[0, 0]
    assert np.array_equal(got, want)


def test_threaded_gemm_is_bit_identical(oracle):
    # the all-core CPU baseline runs the same per-row computation on threads
    rng = np.random.default_rng(12)
    x = rng.standard_normal((37, 160)).astype(np.float32)
    w = rng.integers(-127, 128, (29, 160), dtype=np.int8)
    scale = rng.uniform(0.002, 0.02, 29).astype(np.float32)
    zero = rng.integers(-3, 4, 29).astype(np.int32)
    want = oracle.int8_gemm(x, w, scale, zero)
    for threads in (1, 3, 8):
        got = oracle.int8_gemm_threads(x, w, scale, zero, threads)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_finish_f32_equals_gemm_and_f16_is_one_rounding(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((9, 96)).astype(np.float32)
    w = rng.integers(-127, 128, (13, 96), dtype=np.int8)
    scale = rng.uniform(0.002, 0.02, 13).astype(np.float32)
    zero = rng.integers(-3, 4, 13).astype(np.int32)
    bias = rng.standard_normal(13).astype(np.float32)
    codes, rs, total = oracle.quantize_rows(x)
    acc = oracle.int8_acc(codes, w)
    o32, o16 = oracle.w8a8_finish(acc, total, rs, scale, zero)
    assert np.array_equal(o32, oracle.int8_gemm(x, w, scale, zero))
    assert np.array_equal(o16, o32.astype(np.float16).view(np.uint16))
    b32, b16 = oracle.w8a8_finish(acc, total, rs, scale, zero, bias)
    assert np.array_equal(b32, (o32 + bias[None, :]).astype(np.float32))
    assert np.array_equal(b16, b32.astype(np.float16).view(np.uint16))


# -- W8A16 -----------------------------------------------------------------------


def test_w8a16_f64_matches_numpy(oracle):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 160)).astype(np.float16)
    w = rng.integers(-127, 128, (7, 160), dtype=np.int8)
    s = rng.uniform(0.002, 0.02, 7).astype(np.float16)
    b = rng.standard_normal(7).astype(np.float16)
    got = oracle.w8a16_f64(x, w, s, b)
    want = (x.astype(np.float64) @ w.astype(np.float64).T) * s.astype(np.float64) + b.astype(np.float64)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_w8a16_gemm_exact_on_integers_and_within_tolerance(oracle):
    # integer-valued case: every product and sum is exact in f32 and f16
    x = np.arange(-8, 8, dtype=np.float16).reshape(1, 16)
    w = np.arange(16 * 3, dtype=np.int64).reshape(3, 16).astype(np.int8) - 20
    s = np.ones(3, np.float16)
    got = oracle.w8a16_gemm(x, w, s)
    want = (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float16)
    assert np.array_equal(got, want)
    # random case at a decode shape: the specified 1e-2 tolerance vs f64
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 4096)).astype(np.float16)
    w = rng.integers(-127, 128, (64, 4096), dtype=np.int8)
    s = rng.uniform(0.002, 0.02, 64).astype(np.float16)
    ref = oracle.w8a16_f64(x, w, s)
    got = oracle.w8a16_gemm(x, w, s).astype(np.float64)
    assert tolerance.rel_err(got, ref, truth=False) <= tolerance.FP16_REL_TOL
    # negative control: a 2% scale error on one channel must fail the bar
    bad = got.copy()
    bad[:, 5] *= 1.02
    assert tolerance.rel_err(bad, ref, truth=False) > tolerance.FP16_REL_TOL


# -- ConvRot Hadamard (convrot.rs:121-149, tests :169-220) -----------------------


def test_hadamard_base_and_sign_rule(oracle):
    h4 = oracle.hadamard(4) * 2
    for a in range(4):
        for b in range(4):
            assert h4[a, b] == (-1.0 if a ^ b == 3 else 1.0)
    h16 = oracle.hadamard(16) * 4
    assert np.array_equal(h16, np.kron(h4, h4))  # Kronecker power


def test_hadamard_symmetric_involutory_and_sylvester_magnitudes(oracle):
    import scipy.linalg
    h = oracle.hadamard(256)
    assert np.array_equal(h, h.T)
    assert np.max(np.abs(h @ h - np.eye(256))) < 1e-4
    assert np.array_equal(np.abs(h), np.abs(scipy.linalg.hadamard(256) / 16.0))


def test_rotation_cancels_around_a_float_matmul(oracle):
    # convrot.rs:192-220, plus a 256-group random case
    x = np.array([[1.0, 2.0, -1.0, 0.5], [0.25, -0.5, 1.5, -2.0]], np.float32)
    w = np.array([[0.5, -1.0, 0.25, 2.0], [1.0, 0.0, -0.5, 0.75]], np.float32)
    xr, wr = oracle.rotate(x, 4), oracle.rotate(w, 4)
    assert np.max(np.abs(x[:1] @ w.T - xr[:1] @ wr.T)) < 1e-4
    rng = np.random.default_rng(6)
    x = rng.standard_normal((3, 512)).astype(np.float32)
    w = rng.standard_normal((5, 512)).astype(np.float32)
    assert np.max(np.abs(x @ w.T - oracle.rotate(x) @ oracle.rotate(w).T)) < 1e-3
