"""Shared W4A16 test data: the reference's synthetic pack-quantized weights
(crates/minicpm-v/src/quant.rs:419-462) and random ones, packed as the
checkpoint stores them (two values per byte, low nibble first, plus 8)."""
import numpy as np
import torch


def bf16_bits(values):
    """float32 -> bf16 bit patterns, round to nearest even (torch's cast)."""
    return torch.from_numpy(np.ascontiguousarray(values, dtype=np.float32)).to(torch.bfloat16) \
        .view(torch.int16).numpy().view(np.uint16)


def bf16_value(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def pack_int4(q):
    """int values in [-8, 7], [rows][width] -> uint8 [rows][width / 2]."""
    n = (np.asarray(q, dtype=np.int16) + 8).astype(np.uint8)
    return (n[:, 0::2] & 0xF) | ((n[:, 1::2] & 0xF) << 4)


def reference_synthetic(out, input, group=128):
    """quant.rs:419-462: q = ((r*13 + c*5) % 15) - 7, scale = bf16(0.008 +
    ((r*31 + g*7) % 17) * 0.0007); returns (packed, scale bits, q, stored scales)."""
    r = np.arange(out)[:, None]
    c = np.arange(input)[None, :]
    q = ((r * 13 + c * 5) % 15) - 7
    g = np.arange(input // group)[None, :]
    scale = 0.008 + ((r * 31 + g * 7) % 17).astype(np.float32) * np.float32(0.0007)
    bits = bf16_bits(scale.astype(np.float32))
    return pack_int4(q), bits, q, bf16_value(bits)


def reference_activations(m, input):
    """quant.rs:484-491: x = ((i % 29) - 14) * 0.05 for 21 rows, cast to f16."""
    i = np.arange(21 * input)
    x = (((i % 29).astype(np.float32) - 14.0) * np.float32(0.05)).astype(np.float16).reshape(21, input)
    return x[:m]


def random_case(rng, rows, width, columns, group=128, bias=False):
    x = rng.standard_normal((rows, width)).astype(np.float16)
    q = rng.integers(-8, 8, (columns, width))
    scale = bf16_bits(rng.uniform(0.002, 0.03, (columns, width // group)).astype(np.float32))
    b = rng.standard_normal(columns).astype(np.float16) if bias else None
    return x, pack_int4(q), scale, b
