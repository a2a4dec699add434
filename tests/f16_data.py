"""Inputs of the reference's fp16 GEMV tests, restated
(crates/breeze-tts/src/metal_depth_tests.rs:16-80 and the probe
prototypes/tts-gemv/src/main.rs:12-40)."""
import numpy as np

# (rows, k, n) of metal_depth_tests.rs:20-26
DEPTH_SHAPES = [(4, 32, 7), (4, 96, 65), (8, 1024, 256), (64, 96, 65), (4, 8192, 1024)]
# (k, n) of the probe, prototypes/tts-gemv/src/main.rs:12-18
PROBE_SHAPES = [(1024, 256), (1024, 1024), (1024, 8192), (8192, 1024), (2048, 6144)]


def depth_x(rows: int, k: int) -> np.ndarray:
    """f32 values ((i * 17 % 97) - 48) / 139.13 over rows * k (metal_depth_tests.rs:34-36)."""
    i = np.arange(rows * k, dtype=np.int64)
    return (((i * 17 % 97).astype(np.float32) - np.float32(48.0)) / np.float32(139.13)).reshape(rows, k)


def depth_w(k: int, n: int) -> np.ndarray:
    """f32 values ((i * 13 % 89) - 44) / 251.31 over n * k, laid out [n, k]
    (metal_depth_tests.rs:53-55, the output-major case)."""
    i = np.arange(k * n, dtype=np.int64)
    return (((i * 13 % 89).astype(np.float32) - np.float32(44.0)) / np.float32(251.31)).reshape(n, k)


def depth_tolerance(expected: np.ndarray) -> np.ndarray:
    """|actual - expected| < 0.002 + |expected| * 0.001 (metal_depth_tests.rs:74-76)."""
    return 0.002 + np.abs(expected) * 0.001
