"""ConvRot host-side pieces on the CPU: the rotation matrix and the layer's
guards (crates/qwen-image/src/convrot.rs:12-160, tests :169-220)."""
import numpy as np
import pytest

from omni_int8 import convrot


@pytest.mark.parametrize("size", [4, 16, 64, 256])
def test_hadamard_equals_the_oracle_and_its_sign_rule(oracle, size):
    h = convrot.hadamard(size)
    assert np.array_equal(h, oracle.hadamard(size))
    scale = np.float32(2.0 ** -((size.bit_length() - 1) // 2))
    for r in range(0, size, max(1, size // 16)):
        for c in range(size):
            neg = convrot.sign_negative(r, c, size)
            assert neg == bool(oracle.L.oracle_hadamard_sign_negative(r, c, size))
            assert h[r, c] == (-scale if neg else scale)


def test_hadamard_is_symmetric_and_involutory():
    # convrot.rs:169-190
    h = convrot.hadamard(convrot.GROUP)
    assert np.array_equal(h, h.T)
    assert np.abs(h.astype(np.float64) @ h.astype(np.float64) - np.eye(256)).max() < 1e-4


def test_hadamard_is_the_kronecker_power_of_h4():
    # H4[a][b] = -1 iff a ^ b == 3 (convrot.rs:139-140), extended by Kronecker power
    h4 = np.array([[1 if (a ^ b) != 3 else -1 for b in range(4)] for a in range(4)], np.float64)
    k = h4
    for _ in range(3):
        k = np.kron(k, h4)
    assert np.array_equal(convrot.hadamard(256).astype(np.float64) * 16.0, k)


def test_rotation_cancels_around_a_float_matmul():
    # convrot.rs:192-220
    h = convrot.hadamard(4)
    x = np.array([1.0, 2.0, -1.0, 0.5, 0.25, -0.5, 1.5, -2.0], np.float32).reshape(2, 4)
    w = np.array([0.5, -1.0, 0.25, 2.0, 1.0, 0.0, -0.5, 0.75], np.float32).reshape(2, 4)
    direct = x[0] @ w.T
    rotated = (x @ h)[0] @ (w @ h).T
    assert np.abs(direct - rotated).max() < 1e-4


def test_non_power_of_four_group_is_refused():
    # convrot.rs:122 asserts a power of four
    for size in (2, 8, 32, 128, 255):
        with pytest.raises(ValueError):
            convrot.hadamard(size)


def test_layer_refuses_widths_that_do_not_split_into_groups():
    # convrot.rs:39-43
    import torch
    with pytest.raises(ValueError):
        convrot.Int8Linear(300, 2, torch.zeros(150, dtype=torch.int32), torch.ones(2),
                           torch.zeros(2, dtype=torch.int32))
