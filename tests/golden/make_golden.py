"""Writes tests/golden/int8_path.npz: small input/expected-output vectors for
the int8 matmul path, computed by the CPU oracle at fixed seeds.

The reference holds no fixture files for this path; its known answers are
inline (crates/omni-kernel/src/int8_matmul.rs:700-786, prototypes/int8-gemm/
src/main.rs:69-89, crates/qwen-image/src/convrot.rs:169-271). Cases "hand" and
"tile64" restate those inputs; tests/test_golden.py asserts their expected
outputs against the reference's own numbers (-411/127) independently of the
oracle. The other cases are seeded (numpy default_rng) and exist so the GPU
tests can be checked against committed vectors.

Usage: python tests/golden/make_golden.py   (needs `make -C oracle`)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib  # noqa: E402


def w8a8_case(o, name, x, w, scale, zero, bias=None):
    codes, rs, total = o.quantize_rows(x)
    acc = o.int8_acc(codes, w)
    d = {"x": x, "w": w, "scale": scale, "zero": zero, "codes": codes, "row_scale": rs,
         "row_sum": total, "acc": acc, "out": o.int8_gemm(x, w, scale, zero)}
    if bias is not None:
        o32, o16 = o.w8a8_finish(acc, total, rs, scale, zero, bias)
        d.update(bias=bias, out_bias_f32=o32, out_bias_f16=o16)
    return {f"{name}/{k}": v for k, v in d.items()}


def build():
    o = oracle_lib.Oracle()
    arrays = {}

    # int8_matmul.rs:700-732 and :749-786
    arrays.update(w8a8_case(o, "hand", np.array([[1.0, -2.0, 0.5, 4.0]], np.float32),
                            np.array([[1, -2, 3, -4]], np.int8), np.array([0.25], np.float32),
                            np.array([1], np.int32)))
    # int8_matmul.rs:734-747
    x = np.zeros((64, 64), np.float32)
    x[0, :4] = [1.0, -2.0, 0.5, 4.0]
    w = np.zeros((64, 64), np.int8)
    w[0, :4] = [1, -2, 3, -4]
    zero = np.zeros(64, np.int32)
    zero[0] = 1
    arrays.update(w8a8_case(o, "tile64", x, w, np.full(64, 0.25, np.float32), zero))
    # prototypes/int8-gemm/src/main.rs:69-89
    for rows, width, columns in [(5, 12, 6), (17, 36, 14)]:
        i = np.arange(rows * width)
        x = (((i * 17) % 41) - 20).astype(np.float32).reshape(rows, width)
        w = (((np.arange(columns * width) * 13) % 31) - 15).astype(np.int8).reshape(columns, width)
        scale = (0.05 + np.arange(columns, dtype=np.float32) * 0.01).astype(np.float32)
        zero = ((np.arange(columns) % 5) - 2).astype(np.int32)
        arrays.update(w8a8_case(o, f"proto{rows}x{width}x{columns}", x, w, scale, zero))

    # seeded: 16x256x64 (f16-exact activations, nonzero zero points, bias)
    rng = np.random.default_rng(20250)
    x = rng.standard_normal((16, 256)).astype(np.float16).astype(np.float32)
    x[3, 17] *= 40.0                              # an outlier channel
    x[5] = 0.0                                    # an all-zero row (scale floor)
    w = rng.integers(-128, 128, (64, 256), dtype=np.int8)
    scale = rng.uniform(0.002, 0.02, 64).astype(np.float32)
    zero = rng.integers(-3, 4, 64).astype(np.int32)
    bias = rng.standard_normal(64).astype(np.float32)
    arrays.update(w8a8_case(o, "seeded16x256x64", x, w, scale, zero, bias))

    # seeded W8A16 16x256x64 and 1x512x96 (GEMV shape class)
    for rows, width, columns, seed in [(16, 256, 64, 7), (1, 512, 96, 8)]:
        rng = np.random.default_rng(seed)
        x16 = rng.standard_normal((rows, width)).astype(np.float16)
        w = rng.integers(-127, 128, (columns, width), dtype=np.int8)
        s16 = rng.uniform(0.002, 0.02, columns).astype(np.float16)
        b16 = rng.standard_normal(columns).astype(np.float16)
        name = f"w8a16_{rows}x{width}x{columns}"
        arrays.update({f"{name}/x": x16, f"{name}/w": w, f"{name}/scale": s16,
                       f"{name}/bias": b16, f"{name}/ref_f64": o.w8a16_f64(x16, w, s16, b16)})

    # ConvRot group-256 rotation of 4 rows x 512
    rng = np.random.default_rng(9)
    xr = rng.standard_normal((4, 512)).astype(np.float32)
    arrays.update({"rotate/x": xr, "rotate/out": o.rotate(xr, 256)})
    return arrays


def main():
    arrays = build()
    path = os.path.join(HERE, "int8_path.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path}: {len(arrays)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
