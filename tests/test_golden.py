"""Committed golden vectors (tests/golden/int8_path.npz, written by
tests/golden/make_golden.py from the oracle at fixed seeds).

CPU: the reference's own known answers hold in the fixture (checked without
the oracle), the rotation fixture equals the Sylvester-Hadamard product, and
the oracle still reproduces every vector. GPU: the library reproduces them
(bit-exact for W8A8, 1e-2 relative for W8A16)."""
import os

import numpy as np
import pytest
import torch

import omni_int8 as oi
import tolerance

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "int8_path.npz")
W8A8_CASES = ["hand", "tile64", "proto5x12x6", "proto17x36x14", "seeded16x256x64"]
W8A16_CASES = ["w8a16_16x256x64", "w8a16_1x512x96"]


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def case(golden, name):
    p = name + "/"
    return {k[len(p):]: v for k, v in golden.items() if k.startswith(p)}


def test_hand_value_is_the_references(golden):
    # int8_matmul.rs:700-732: codes [32,-64,16,127], acc -300, sum 111,
    # centered -300 - 111*1 = -411, times (4/127) * 0.25 -> -411/127.
    c = case(golden, "hand")
    assert c["codes"].tolist() == [[32, -64, 16, 127]]
    assert c["acc"].tolist() == [[-300]] and c["row_sum"].tolist() == [111]
    assert c["row_scale"][0] == np.float32(4.0) / np.float32(127.0)
    assert abs(float(c["out"][0, 0]) - (-411.0 / 127.0)) < 1e-6


def test_tile64_fixture_is_the_references(golden):
    # int8_matmul.rs:734-747: one live entry, everything else exactly zero.
    c = case(golden, "tile64")
    assert abs(float(c["out"][0, 0]) - (-411.0 / 127.0)) < 1e-6
    rest = c["out"].copy()
    rest[0, 0] = 0.0
    assert not rest.any()


def test_w8a8_vectors_are_integer_consistent(golden):
    # acc and sums follow from the codes by exact integer arithmetic, and the
    # codes lie in range and reproduce x to within half a quantisation step.
    for name in W8A8_CASES:
        c = case(golden, name)
        acc = c["codes"].astype(np.int64) @ c["w"].astype(np.int64).T
        assert np.array_equal(acc, c["acc"]), name
        assert np.array_equal(c["codes"].astype(np.int64).sum(1), c["row_sum"]), name
        err = np.abs(c["codes"] * c["row_scale"][:, None].astype(np.float64) - c["x"])
        assert np.all(err <= 0.5 * c["row_scale"][:, None] * (1 + 1e-6)), name


def test_rotate_fixture_is_sylvester_hadamard(golden):
    # convrot.rs:113-149: the sign rule "odd number of base-4 digits equal to
    # 3 in row ^ col" is the Kronecker power H4 (x) H4 (x) H4 (x) H4 with
    # H4[a,b] = -1 iff a ^ b == 3; the scale is 2^-log4(256) = 1/16.
    h4 = np.ones((4, 4))
    for a in range(4):
        for b in range(4):
            if a ^ b == 3:
                h4[a, b] = -1.0
    h = h4
    for _ in range(3):
        h = np.kron(h, h4)
    h /= 16.0
    x = golden["rotate/x"].astype(np.float64)
    want = (x.reshape(-1, 256) @ h).reshape(x.shape)
    assert np.max(np.abs(golden["rotate/out"] - want)) < 1e-5


def test_oracle_reproduces_every_vector(golden):
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "make_golden", os.path.join(os.path.dirname(GOLDEN), "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    fresh = mg.build()
    assert sorted(fresh) == sorted(golden)
    for k, v in fresh.items():
        assert v.dtype == golden[k].dtype and np.array_equal(v.view(np.uint8), golden[k].view(np.uint8)), k


# -- GPU ------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("name", W8A8_CASES)
def test_gpu_w8a8_matches_golden(golden, name):
    c = case(golden, name)
    dev = "cuda"
    x = torch.from_numpy(c["x"]).to(dev)
    w = torch.from_numpy(c["w"]).to(dev)
    scale = torch.from_numpy(c["scale"]).to(dev)
    zero = torch.from_numpy(c["zero"]).to(dev)
    out = oi.try_int8_gemm(x, w.view(torch.int32).reshape(-1), scale, zero)
    codes, rs, total = oi.quantize_rows(x)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), c["out"].view(np.uint32))
    assert np.array_equal(codes.cpu().numpy(), c["codes"])
    assert np.array_equal(rs.cpu().numpy().view(np.uint32), c["row_scale"].view(np.uint32))
    assert np.array_equal(total.cpu().numpy(), c["row_sum"])
    for low in (oi.OMNI_LOWERING_MFMA, oi.OMNI_LOWERING_SCALAR):
        if low == oi.OMNI_LOWERING_MFMA and c["x"].shape[1] % 16:
            continue
        o, acc = oi.w8a8_gemm(codes, rs, total, w, scale, zero, acc_dump=True, lowering=low)
        torch.cuda.synchronize()
        assert np.array_equal(acc.cpu().numpy(), c["acc"]), (name, low)
        assert np.array_equal(o.cpu().numpy().view(np.uint32), c["out"].view(np.uint32)), (name, low)
    if "bias" in c:
        b = torch.from_numpy(c["bias"]).to(dev)
        o32 = oi.w8a8_gemm(codes, rs, total, w, scale, zero, bias=b)
        o16 = oi.w8a8_gemm(codes, rs, total, w, scale, zero, bias=b, out_dtype=torch.float16)
        torch.cuda.synchronize()
        assert np.array_equal(o32.cpu().numpy().view(np.uint32), c["out_bias_f32"].view(np.uint32))
        assert np.array_equal(o16.cpu().numpy().view(np.uint16), c["out_bias_f16"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", W8A16_CASES)
def test_gpu_w8a16_matches_golden(golden, name):
    c = case(golden, name)
    t = {k: torch.from_numpy(c[k]).to("cuda") for k in ("x", "w", "scale", "bias")}
    y = oi.w8a16_linear(t["x"], t["w"], t["scale"], t["bias"])
    torch.cuda.synchronize()
    err = tolerance.rel_err(y.cpu().numpy(), c["ref_f64"])
    assert err <= tolerance.FP16_REL_TOL, (name, err)
