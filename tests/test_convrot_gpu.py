"""ConvRot rotation + quantisation + GEMM on the GPU against the oracle.

The reference rotates with an f32 matmul (crates/qwen-image/src/convrot.rs:
113-119), the oracle with an f32 dot in j order; the kernel with a radix-4
fast transform. All three are the same linear map rounded differently, so
the bar is: row scales within a few ulp; codes equal except where the
rotated value sits within rounding of a half-way point, and there by at
most one; layer outputs within the reference test's tolerance (1e-2,
convrot.rs:266) and the north_star one (1e-2 relative, fp16 out).
"""
import numpy as np
import pytest
import torch

import omni_int8 as oi
from omni_int8 import convrot
import tolerance

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    assert oi.arch_supported(torch.cuda.current_device()), "device is not gfx950"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def exact_rotation(x):
    """f64 rotation of f32 inputs: products are exact, the 256-term sums
    carry ~1e-16 relative error."""
    h = convrot.hadamard(256).astype(np.float64)
    rows, width = x.shape
    return (x.astype(np.float64).reshape(-1, 256) @ h).reshape(rows, width)


def fwht_band(x, scale, roundings=12):
    """Where the kernel's codes may differ from the exact rotation's, in
    units of r / row_scale: the fast transform's error bound on u = 16 r
    (12 roundings' worth, 12 * 2^-24 * the group's sum |x|, plus 1 % for
    second-order terms) over 16 row_scale, plus the row scales' own few-ulp
    disagreement (2e-6 relative of |q| <= 127.5). roundings=255 gives the
    bound of a serial 256-term f32 dot (the oracle's matmul order)."""
    rows, width = x.shape
    g = np.abs(x.astype(np.float64)).reshape(rows, width // 256, 256).sum(axis=2)
    bound_u = np.repeat(g, 256, axis=1).reshape(rows, width) * roundings * 2.0 ** -24 * 1.01
    return bound_u / (16.0 * scale[:, None].astype(np.float64)) + 127.5 * 2e-6


def check_codes(codes, scale, total, r_ref, oracle_scale, band):
    """codes/scale/total from the GPU against a rotation r_ref (f64) quantised
    with the reference rule: equal, except by one inside `band` of a half-way
    point."""
    # the row peaks of two roundings of one rotation: a few ulp apart
    np.testing.assert_allclose(scale, oracle_scale, rtol=2e-6, atol=0)
    q = r_ref / scale[:, None].astype(np.float64)
    want = np.clip(np.sign(q) * np.floor(np.abs(q) + 0.5), -128, 127)
    want = np.where(np.isnan(q), 0, want).astype(np.int64)
    got = codes.astype(np.int64)
    diff = np.abs(got - want)
    assert diff.max() <= 1
    if diff.any():
        near = np.abs(np.abs(q) - np.floor(np.abs(q)) - 0.5)
        assert np.all(near[diff == 1] <= band[diff == 1]), near[diff == 1].max()
    assert np.array_equal(total, got.sum(axis=1))


def check_bit_exact(oracle, x32, codes, scale, total):
    """The kernel's codes, row scales and sums equal the oracle's restatement
    of its fast transform followed by the reference quantisation, bit for bit."""
    ocodes, oscale, ototal = oracle.convrot_quantize_fwht(x32)
    assert np.array_equal(codes, ocodes)
    assert np.array_equal(scale.view(np.uint32), oscale.view(np.uint32))
    assert np.array_equal(total, ototal)


# widths of 1-64 groups take the packed-rows kernel (1-4 waves, 1-16 rows per
# workgroup); wider rows take the four-wave two-pass kernel (81 groups: two
# passes, the second mostly idle)
@pytest.mark.parametrize("rows,width", [(1, 256), (7, 512), (33, 3072), (5, 4096), (3, 2304),
                                        (4, 4352), (2, 12288), (1, 16384), (37, 256), (9, 768),
                                        (3, 20736)])
@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_fused_rotation_quantisation_matches_the_oracle(oracle, rows, width, dtype):
    rng = np.random.default_rng(rows * 7 + width)
    x = rng.standard_normal((rows, width)).astype(dtype)
    codes, scale, total = convrot.convrot_quantize_rows(dev(x))
    codes, scale, total = host(codes), host(scale), host(total)
    x32 = x.astype(np.float32)
    check_bit_exact(oracle, x32, codes, scale, total)
    # and against the reference's own f32 matmul rotation (the oracle's dot
    # order) and the exact rotation: equal outside the transform's band
    r32 = oracle.rotate(x32)
    _, o_scale, _ = oracle.quantize_rows(r32)
    band = fwht_band(x32, scale) + fwht_band(x32, scale, roundings=255)
    check_codes(codes, scale, total, r32.astype(np.float64), o_scale, band)
    check_codes(codes, scale, total, exact_rotation(x32), o_scale, fwht_band(x32, scale))


def test_outlier_channels_and_strided_rows(oracle):
    # config 4's activations: 1% of channels scaled x20; rows with a stride
    rng = np.random.default_rng(4)
    rows, width, ld = 19, 3072, 3072 + 256
    x = rng.standard_normal((rows, ld)).astype(np.float16)
    hot = rng.choice(width, width // 100, replace=False)
    x[:, hot] *= 20
    xt = dev(x)[:, :width]
    assert xt.stride(0) == ld
    codes, scale, total = convrot.convrot_quantize_rows(xt)
    xs = x[:, :width].astype(np.float32)
    check_bit_exact(oracle, xs, host(codes), host(scale), host(total))
    _, o_scale, _ = oracle.quantize_rows(oracle.rotate(xs))
    check_codes(host(codes), host(scale), host(total), exact_rotation(xs), o_scale,
                fwht_band(xs, host(scale)))


def test_nan_zero_and_tiny_rows(oracle):
    x = np.zeros((4, 512), np.float32)
    x[0, 3] = np.nan                       # the whole first group turns NaN -> codes 0
    x[0, 300] = 1.0
    x[2] = np.linspace(-1e-26, 1e-26, 512, dtype=np.float32)  # row scale below 2^-90
    x[3] = np.linspace(-3.0, 5.0, 512, dtype=np.float32)
    codes, scale, total = convrot.convrot_quantize_rows(dev(x))
    codes, scale, total = host(codes), host(scale), host(total)
    check_bit_exact(oracle, x, codes, scale, total)
    r = oracle.rotate(x)
    o_codes, o_scale, o_sum = oracle.quantize_rows(r)
    assert np.all(codes[0, :256] == 0) and np.all(o_codes[0, :256] == 0)
    assert np.array_equal(codes[1], o_codes[1]) and scale[1] == np.float32(1e-30)
    check_codes(codes[2:], scale[2:], total[2:], exact_rotation(x[2:]), o_scale[2:],
                fwht_band(x[2:], scale[2:]))
    check_codes(codes[:1, 256:], scale[:1], codes[:1, 256:].astype(np.int64).sum(1),
                exact_rotation(x[:1, 256:]), o_scale[:1], fwht_band(x[:1, 256:], scale[:1]))


def test_reference_linear_case(oracle):
    # convrot.rs:222-271: 2 x 256 input, 2 outputs, scale [0.05, 0.2], zero [0, 2]
    rows, width, columns = 2, 256, 2
    x = ((np.arange(rows * width) % 17).astype(np.float32) - 8.0) * 0.125
    x = x.reshape(rows, width)
    w = (((np.arange(columns * width) * 13) % 31) - 15).astype(np.int8).reshape(columns, width)
    scale = np.array([0.05, 0.2], np.float32)
    zero = np.array([0, 2], np.int32)
    layer = convrot.Int8Linear(width, columns, dev(oracle.pack_i8(w)), dev(scale), dev(zero),
                               precision=torch.float32)
    got = host(layer(dev(x)))
    expected = oracle.dequant_reference(oracle.rotate(x), w, scale, zero)
    assert np.abs(got - expected).max() < 1e-2
    # and the integer route, rotation then the reference's own int8 gemm
    assert np.abs(got - oracle.int8_gemm(oracle.rotate(x), w, scale, zero)).max() < 1e-2


@pytest.mark.parametrize("rows,width,columns", [(64, 3072, 1024), (37, 12288, 640), (4352, 3072, 9216)])
def test_layer_at_diffusion_shapes(oracle, rows, width, columns):
    # BASELINE config 4 (QKV K=3072, N=9216 at M=4352) and the down projection's
    # width; fp16 activations and output (Precision::F16)
    rng = np.random.default_rng(rows + width)
    x = rng.standard_normal((rows, width)).astype(np.float16)
    w = rng.integers(-127, 128, (columns, width), dtype=np.int8)
    scale = rng.uniform(0.002, 0.02, columns).astype(np.float32)
    zero = rng.integers(-2, 3, columns).astype(np.int32)
    layer = convrot.Int8Linear(width, columns, dev(oracle.pack_i8(w)), dev(scale), dev(zero))
    got = host(layer(dev(x).reshape(1, rows, width)))
    assert got.shape == (1, rows, columns) and got.dtype == np.float16
    sample = rng.choice(rows, min(rows, 8), replace=False)
    xs = x[sample].astype(np.float32)
    ref = oracle.int8_gemm(oracle.rotate(xs), w, scale, zero).astype(np.float16)
    assert tolerance.rel_err(got[0, sample], ref.astype(np.float64), truth=False) <= tolerance.FP16_REL_TOL


def test_fused_path_equals_rotate_then_quantize_on_the_gpu():
    # the unfused reference route on the GPU: f32 matmul by H, then quantize_rows
    rng = np.random.default_rng(11)
    x = rng.standard_normal((256, 4096)).astype(np.float32)
    h = dev(convrot.hadamard(256))
    xt = dev(x)
    r = (xt.reshape(-1, 256) @ h).reshape(256, 4096)
    c_ref, s_ref, _ = oi.quantize_rows(r)
    c, s, t = convrot.convrot_quantize_rows(xt)
    assert torch.allclose(s, s_ref, rtol=2e-6, atol=0)
    d = (c.int() - c_ref.int()).abs()
    assert int(d.max()) <= 1 and float(d.float().mean()) < 1e-3
    assert torch.equal(t, c.int().sum(dim=1))


def test_guards():
    x = torch.zeros((2, 300), device="cuda")
    with pytest.raises(ValueError):
        convrot.convrot_quantize_rows(x)  # width % 256 != 0: not handled
    layer = convrot.Int8Linear(256, 2, torch.zeros(128, dtype=torch.int32, device="cuda"),
                               torch.ones(2, device="cuda"), torch.zeros(2, dtype=torch.int32, device="cuda"))
    with pytest.raises(ValueError):
        layer(torch.zeros((2, 512), device="cuda"))  # width != the layer's (convrot.rs:84)
    bad = convrot.Int8Linear(256, 2, torch.zeros(100, dtype=torch.int32, device="cuda"),
                             torch.ones(2, device="cuda"), torch.zeros(2, dtype=torch.int32, device="cuda"))
    with pytest.raises(RuntimeError):
        bad(torch.zeros((2, 256), device="cuda"))  # packed length disagrees: project() panics


def test_layer_loaded_from_a_checkpoint(oracle, tmp_path):
    # ConvRotFile::linear (convrot.rs:30-67) feeding the GPU layer, checked
    # against the oracle route on the same tensors
    from safetensors.numpy import save_file
    rng = np.random.default_rng(21)
    name, output, input = "transformer_blocks.3.ff.net.0.proj", 48, 768
    q = rng.integers(-127, 128, (output, input), dtype=np.int8)
    scale = rng.uniform(0.002, 0.02, output).astype(np.float32)
    zero = rng.integers(-2, 3, output).astype(np.int8)
    save_file({f"{name}._weight_qdata": q, f"{name}._weight_scale": scale,
               f"{name}._weight_zero_point": zero}, str(tmp_path / convrot.FILE_NAME))
    layer = convrot.ConvRotFile.open(str(tmp_path)).linear(name, input, output, precision=torch.float32)
    x = rng.standard_normal((5, input)).astype(np.float32)
    got = host(layer(dev(x)))
    want = oracle.int8_gemm(oracle.rotate(x), q, scale, zero.astype(np.int32))
    assert tolerance.rel_err(got, want.astype(np.float64), truth=False) <= tolerance.FP16_REL_TOL
