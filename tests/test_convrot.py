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


# -- the kernel's fast transform as the oracle restates it -------------------------


def test_fast_transform_is_the_hadamard_on_unit_vectors(oracle):
    # Every op of the transform on a unit vector is exact, so the outputs must
    # be column j of 16 H exactly: a wrong sign, index or stage order fails.
    eye = np.eye(256, dtype=np.float32)
    u = oracle.convrot_fwht(eye)
    assert np.array_equal(u, convrot.hadamard(256) * np.float32(16.0))
    # and group by group along a row: group g of a 3-group row sees only its own slice
    x = np.zeros((256, 768), np.float32)
    x[:, 256:512] = eye
    u = oracle.convrot_fwht(x)
    assert not u[:, :256].any() and not u[:, 512:].any()
    assert np.array_equal(u[:, 256:512], convrot.hadamard(256) * np.float32(16.0))


def _fwht_bound(x):
    """First-order forward error bound of the four radix-4 stages on u = 16 r:
    each stage adds at most 3 roundings to every partial sum, whose magnitude
    is at most the sum of |x| over the inputs feeding it, and the later stages
    spread an error over disjoint input sets of the group, so the total is
    12 * 2^-24 * sum_group |x| (plus second-order terms: slack 1 %)."""
    rows, width = x.shape
    g = np.abs(x.astype(np.float64)).reshape(rows, width // 256, 256).sum(axis=2)
    return np.repeat(g, 256, axis=1).reshape(rows, width) * 12.0 * 2.0 ** -24 * 1.01


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_fast_transform_within_its_error_bound_of_the_exact_rotation(oracle, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((64, 3072)).astype(np.float32)
    x[:, rng.choice(3072, 30, replace=False)] *= 20  # outlier channels
    x[5] = x[5].astype(np.float16).astype(np.float32)  # f16-valued inputs
    x[7] *= np.float32(1e-20)  # tiny magnitudes
    x[9] = np.abs(x[9])  # no cancellation
    u = oracle.convrot_fwht(x).astype(np.float64)
    h16 = convrot.hadamard(256).astype(np.float64) * 16.0
    exact = (x.astype(np.float64).reshape(-1, 256) @ h16).reshape(x.shape)
    err = np.abs(u - exact)
    bound = _fwht_bound(x)
    assert np.all(err <= bound)
    # the bound is not vacuous: the transform does round
    assert err.max() > 0


def test_fast_transform_codes_follow_the_reference_rule(oracle):
    # The codes from the fast transform are the reference quantisation of
    # r = u / 16: checked against quantize_rows on r (which the reference's
    # own cases pin), bit for bit, including the row scales and sums.
    rng = np.random.default_rng(4)
    x = rng.standard_normal((40, 1024)).astype(np.float32)
    x[3] = 0.0
    x[4] *= np.float32(1e-28)  # row scale at the 1e-30 floor
    codes, scale, total = oracle.convrot_quantize_fwht(x)
    r = oracle.convrot_fwht(x) * np.float32(0.0625)
    rc, rs, rt = oracle.quantize_rows(r)
    assert np.array_equal(codes, rc) and np.array_equal(total, rt)
    assert np.array_equal(scale.view(np.uint32), rs.view(np.uint32))


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


# -- checkpoint loader (convrot.rs:15-68, src/weights.rs:301-304, 429-462) -------

def _write_layer(path, name, output, input, seed=0, scale_dtype=np.float32, extra=None):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(seed)
    t = {f"{name}._weight_qdata": rng.integers(-128, 128, (output, input), dtype=np.int8),
         f"{name}._weight_scale": rng.uniform(0.002, 0.02, output).astype(scale_dtype),
         f"{name}._weight_zero_point": rng.integers(-3, 4, output).astype(np.int8)}
    t.update(extra or {})
    save_file(t, path, metadata={"format": "convrot_hadamard_v1"})
    return t


def test_loader_reads_a_layer_written_by_the_safetensors_library(tmp_path):
    import torch
    name = "transformer_blocks.0.attn.to_q"
    t = _write_layer(str(tmp_path / convrot.FILE_NAME), name, 8, 512)
    f = convrot.ConvRotFile.open(str(tmp_path))
    assert f is not None and f.weights.metadata["format"] == "convrot_hadamard_v1"
    layer = f.linear(name, 512, 8, precision=torch.float16, device="cpu")
    q = t[f"{name}._weight_qdata"]
    assert layer.packed.dtype == torch.int32 and layer.packed.numel() == 8 * 512 // 4
    # the packed words are the row-major int8 bytes (convrot.rs:151-160)
    assert np.array_equal(layer.packed.numpy().view(np.int8).reshape(8, 512), q)
    assert np.array_equal(layer.scale.numpy(), t[f"{name}._weight_scale"])
    assert np.array_equal(layer.zero.numpy(), t[f"{name}._weight_zero_point"].astype(np.int32))


def test_loader_raw_views_match_every_tensor(tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(3)
    t = {"a": rng.integers(-128, 128, (3, 5, 7), dtype=np.int8),
         "b": rng.standard_normal((4, 6)).astype(np.float32),
         "c": rng.standard_normal(9).astype(np.float32)}
    path = str(tmp_path / "x.safetensors")
    save_file(t, path)
    f = convrot.SafetensorsFile(path)
    assert f.names() == ["a", "b", "c"]
    shape, a = f.raw_i8("a")
    assert shape == (3, 5, 7) and np.array_equal(a.reshape(shape), t["a"])
    for k in ("b", "c"):
        shape, v = f.raw_f32(k)
        assert shape == t[k].shape and np.array_equal(v.reshape(shape), t[k])
    with pytest.raises(convrot.CheckpointError, match="expected I8"):
        f.raw_i8("b")
    with pytest.raises(convrot.CheckpointError, match="missing tensor"):
        f.raw_f32("d")


def test_loader_refusals(tmp_path):
    name = "blk.mlp.down"
    assert convrot.ConvRotFile.open(str(tmp_path)) is None  # no file: None (convrot.rs:22-24)
    path = str(tmp_path / convrot.FILE_NAME)
    _write_layer(path, name, 4, 256)
    f = convrot.ConvRotFile.open(str(tmp_path))
    with pytest.raises(convrot.ConfigError):
        f.linear(name, 256, 5, device="cpu")      # scale/zero length != output
    with pytest.raises(convrot.ConfigError):
        f.linear(name, 512, 4, device="cpu")      # qdata shape != [output, input]
    with pytest.raises(convrot.ConfigError):
        f.linear(name, 260, 4, device="cpu")      # input not a multiple of 256
    with pytest.raises(convrot.CheckpointError):
        f.linear("other", 256, 4, device="cpu")   # missing tensors
    _write_layer(path, name, 4, 256, scale_dtype=np.float16)
    with pytest.raises(convrot.CheckpointError, match="expected F32"):
        convrot.ConvRotFile.open(str(tmp_path)).linear(name, 256, 4, device="cpu")


def test_loader_rejects_a_corrupt_file(tmp_path):
    path = tmp_path / "bad.safetensors"
    path.write_bytes((10 ** 6).to_bytes(8, "little") + b"{}")
    with pytest.raises(convrot.CheckpointError):
        convrot.SafetensorsFile(str(path))
    header = b'{"w": {"dtype": "I8", "shape": [4, 4], "data_offsets": [0, 64]}}'
    path.write_bytes(len(header).to_bytes(8, "little") + header + bytes(16))
    with pytest.raises(convrot.CheckpointError, match="outside"):
        convrot.SafetensorsFile(str(path))
    header = b'{"w": {"dtype": "I8", "shape": [4, 5], "data_offsets": [0, 16]}}'
    path.write_bytes(len(header).to_bytes(8, "little") + header + bytes(16))
    with pytest.raises(convrot.CheckpointError, match="payload"):
        convrot.SafetensorsFile(str(path)).raw_i8("w")
