"""W4A16 oracle pins on the CPU (crates/minicpm-v/src/quant.rs)."""
import numpy as np
import torch

import w4a16_data as wd


def test_unpack_int4_every_byte(oracle):
    # quant.rs:22-29: low nibble first, unsigned nibble minus 8 (8 -> 0, 0 -> -8)
    b = np.arange(256, dtype=np.uint8)
    v = oracle.unpack_int4(b).reshape(256, 2)
    for byte in range(256):
        assert v[byte, 0] == (byte & 0xF) - 8 and v[byte, 1] == (byte >> 4) - 8
    assert oracle.unpack_int4(np.array([0x88], np.uint8)).tolist() == [0, 0]
    assert oracle.unpack_int4(np.array([0x0F], np.uint8)).tolist() == [7, -8]


def test_bf16_decode_every_pattern_against_torch(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    got = np.array([oracle.L.oracle_bf16_to_f32(int(b)) for b in bits[::97]], np.float32)
    want = want[::97]
    # a signalling NaN comes back quieted through the ctypes float return
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_pack_round_trips_through_the_oracle(oracle):
    rng = np.random.default_rng(2)
    q = rng.integers(-8, 8, (5, 64))
    assert np.array_equal(oracle.unpack_int4(wd.pack_int4(q)).reshape(5, 64), q)


def test_synthetic_weights_dequantise_exactly(oracle):
    # quant.rs:419-462: the packed codes and bf16 scales reproduce q * scale
    packed, bits, q, scale = wd.reference_synthetic(64, 512)
    w = oracle.w4a16_dequant(packed, bits, 64, 512)
    want = q.astype(np.float32) * np.repeat(scale, 128, axis=1)
    assert np.array_equal(w, want)
    w16 = oracle.w4a16_dequant(packed, bits, 64, 512, f16_round=True)
    assert np.array_equal(w16, want.astype(np.float16).astype(np.float32))


def test_route_meets_the_reference_tolerance(oracle):
    # quant.rs:466-503 at its own shapes (tolerance 5e-2 absolute vs f64)
    for out, input, m in [(512, 2048, 21), (2048, 512, 21), (512, 2048, 1)]:
        packed, bits, q, scale = wd.reference_synthetic(out, input)
        x = wd.reference_activations(m, input)
        truth = oracle.w4a16_f64(x, packed, bits)
        exact = x.astype(np.float64) @ (q.astype(np.float64) * np.repeat(scale, 128, axis=1)).T
        assert np.abs(truth - exact).max() < 1e-9
        route = oracle.w4a16_gemm(x, packed, bits).astype(np.float64)
        assert np.abs(route - truth).max() < 5e-2
