"""W4A16 (MiniCPM-V pack-quantized int4, group 128, bf16 scales) on the GPU.

The reference dequantises inside Burn/cubek's quantized matmul on the GPU and
at load on the CPU (crates/minicpm-v/src/quant.rs:145-201); both are checked
by its own test against an f64 product with a 5e-2 absolute tolerance
(quant.rs:466-503). Here: that test's synthetic weights and shapes, and
random cases over every kernel path (GEMV, skinny, tiled prefill) against
the f64 truth at 1e-2 relative and the oracle's dequantise-then-dot route.
"""
import numpy as np
import pytest
import torch

import omni_int8 as oi
import tolerance
import w4a16_data as wd

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    assert oi.arch_supported(torch.cuda.current_device()), "device is not gfx950"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run(x, packed, bits, b=None, group=128):
    scale = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()
    y = oi.w4a16_linear(dev(x), dev(packed), scale, None if b is None else dev(b), group=group)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("out,input,m", [(512, 2048, 21), (2048, 512, 21), (512, 2048, 1),
                                         (512, 2048, 4), (2048, 512, 130)])
def test_reference_synthetic_case(oracle, out, input, m):
    packed, bits, q, scale = wd.reference_synthetic(out, input)
    if m <= 21:
        x = wd.reference_activations(m, input)
    else:
        x = np.tile(wd.reference_activations(21, input), (m // 21 + 1, 1))[:m]
    got = run(x, packed, bits).astype(np.float64)
    truth = oracle.w4a16_f64(x, packed, bits)
    assert np.abs(got - truth).max() < 5e-2            # the reference's own bar
    assert tolerance.rel_err(got, truth) <= tolerance.FP16_REL_TOL


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 16, 33, 64, 65, 300])
@pytest.mark.parametrize("width,columns,group", [(2048, 512, 128), (512, 2048, 128), (4096, 77, 128),
                                                 (1536, 130, 64), (96, 9, 32), (14336, 40, 128)])
def test_every_path_random(oracle, rows, width, columns, group):
    rng = np.random.default_rng(rows * 7 + width + columns + group)
    x, packed, bits, b = wd.random_case(rng, rows, width, columns, group, bias=columns % 2 == 1)
    got = run(x, packed, bits, b, group).astype(np.float64)
    truth = oracle.w4a16_f64(x, packed, bits, group, b)
    assert tolerance.rel_err(got, truth) <= tolerance.FP16_REL_TOL, (rows, width, columns, group)
    route = oracle.w4a16_gemm(x, packed, bits, group, b).astype(np.float64)
    assert tolerance.rel_err(got, route, truth=False) <= tolerance.FP16_REL_TOL


@pytest.mark.parametrize("r", ["11", "21", "41", "81", "42", "44", "82"])
def test_gemv_every_rows_per_workgroup(oracle, monkeypatch, r, knobs):
    # OMNI_W4A16_GEMV=<rows per batch><batches per workgroup>; column counts
    # leave the last workgroup's batches partly or wholly past the matrix;
    # one row at K = 4096 / 14336 with group 128 runs the kernels built for
    # those shapes
    knobs.set("OMNI_W4A16_GEMV", r)
    for rows, width, columns, group in ((1, 4096, 37, 32), (4, 2048, 130, 32), (3, 96, 9, 32),
                                        (1, 4096, 37, 128), (1, 14336, 21, 128)):
        rng = np.random.default_rng(rows + width + columns + int(r))
        x, packed, bits, b = wd.random_case(rng, rows, width, columns, group, bias=True)
        got = run(x, packed, bits, b, group).astype(np.float64)
        truth = oracle.w4a16_f64(x, packed, bits, group, b)
        assert tolerance.rel_err(got, truth) <= tolerance.FP16_REL_TOL, (r, rows, width, columns)


@pytest.mark.parametrize("columns", [2048, 2051, 2056, 2063, 14336])
def test_gemv_two_team_build(oracle, columns):
    # one row at K = 4096, group 128, from 4 MB of codes: two 128-lane teams
    # of 8 rows per workgroup; the last workgroup's second team lies partly
    # (2051, 2063) or wholly (2056) past the matrix
    rng = np.random.default_rng(columns)
    x, packed, bits, b = wd.random_case(rng, 1, 4096, columns, 128, bias=True)
    got = run(x, packed, bits, b, 128).astype(np.float64)
    truth = oracle.w4a16_f64(x, packed, bits, 128, b)
    assert tolerance.rel_err(got, truth) <= tolerance.FP16_REL_TOL, columns
    route = oracle.w4a16_gemm(x, packed, bits, 128, b).astype(np.float64)
    assert tolerance.rel_err(got, route, truth=False) <= tolerance.FP16_REL_TOL, columns


def test_integer_inputs_are_exact():
    # integer x and unit scales: every partial sum is an integer below 2^11
    x = np.tile(np.arange(-4, 4, dtype=np.float16), (3, 32))[:, :256].copy()
    q = ((np.arange(6 * 256) % 7) - 3).reshape(6, 256)
    bits = wd.bf16_bits(np.ones((6, 2), np.float32))
    for rows in (3, 9, 70):
        xr = np.tile(x, (rows // 3 + 1, 1))[:rows]
        got = run(xr, wd.pack_int4(q), bits)
        want = (xr.astype(np.int64) @ q.astype(np.int64).T).astype(np.float16)
        assert np.array_equal(got, want), rows


def test_guards():
    x = torch.zeros((2, 200), dtype=torch.float16, device="cuda")
    w = torch.zeros((4, 100), dtype=torch.uint8, device="cuda")
    s = torch.zeros((4, 2), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        oi.w4a16_linear(x, w, s, group=100)   # group % 32 != 0: not handled


@pytest.mark.parametrize("tile", ["1", "2", "4", "5", "6", "10", "16", "17", "18"])
@pytest.mark.parametrize("rows,width,columns,group", [(300, 512, 200, 128), (1024, 1536, 1536, 128),
                                                      (257, 8960, 129, 64), (197, 4096, 640, 256),
                                                      (65, 64, 33, 64), (600, 4096, 700, 128),
                                                      (130, 1536, 96, 32)])
def test_every_prefill_kernel(oracle, monkeypatch, tile, rows, width, columns, group, knobs):
    # OMNI_W4A16_TILE pins one prefill kernel: the tiled GEMMs (1, 2) and the
    # LDS-DMA rings on packed codes (4 = 256 x 128, 5 = 128 x 128, 6 = 256 x 256,
    # 10 = 128 x 128 two per CU, 16 / 17 / 18 = 128 x 256 / 256 x 256 /
    # 256 x 256 with eight waves; group 32 is not a ring case and takes the default); ragged
    # rows/columns, bias, against the f64 truth
    knobs.set("OMNI_W4A16_TILE", tile)
    rng = np.random.default_rng(rows + width + columns + group + int(tile))
    x, packed, bits, b = wd.random_case(rng, rows, width, columns, group, bias=True)
    got = run(x, packed, bits, b, group).astype(np.float64)
    truth = oracle.w4a16_f64(x, packed, bits, group, b)
    assert tolerance.rel_err(got, truth) <= tolerance.FP16_REL_TOL, (tile, rows, width, columns, group)


@pytest.mark.parametrize("tile", ["4", "5", "16", "17", "18"])
def test_ring_integer_inputs_are_exact(monkeypatch, tile, knobs):
    # integer x and unit scales through the rings: every product and f32
    # partial sum is an exact integer, rounded once to f16 as the int64 product is
    knobs.set("OMNI_W4A16_TILE", tile)
    x = np.tile(np.arange(-4, 4, dtype=np.float16), (3, 64))[:, :512].copy()
    q = ((np.arange(70 * 512) % 7) - 3).reshape(70, 512)
    bits = wd.bf16_bits(np.ones((70, 4), np.float32))
    for rows in (3, 130, 300):
        xr = np.tile(x, (rows // 3 + 1, 1))[:rows]
        got = run(xr, wd.pack_int4(q), bits)
        want = (xr.astype(np.int64) @ q.astype(np.int64).T).astype(np.float16)
        assert np.array_equal(got, want), (tile, rows)


@pytest.mark.parametrize("tile", ["0", "4", "18"])
def test_scales_at_an_odd_bf16_offset(oracle, monkeypatch, tile, knobs):
    # The rings copy scales as 4-byte pairs; a scale array starting 2 bytes
    # past a 4-byte boundary (a contiguous view at an odd element) takes the
    # register-staged kernel instead, with the same result bar
    knobs.set("OMNI_W4A16_TILE", tile)
    rng = np.random.default_rng(int(tile) + 11)
    x, packed, bits, b = wd.random_case(rng, 300, 1024, 200, 128, bias=True)
    flat = np.concatenate([np.zeros(1, np.uint16), bits.reshape(-1)])
    big = torch.from_numpy(flat.view(np.int16)).view(torch.bfloat16).cuda()
    scale = big[1:].view(bits.shape)
    assert scale.is_contiguous() and scale.data_ptr() % 4 == 2
    got = oi.w4a16_linear(dev(x), dev(packed), scale, dev(b), group=128)
    torch.cuda.synchronize()
    truth = oracle.w4a16_f64(x, packed, bits, 128, b)
    assert tolerance.rel_err(got.cpu().numpy().astype(np.float64), truth) <= tolerance.FP16_REL_TOL


@pytest.mark.parametrize("seed", range(12))
def test_default_routing_random_shapes(oracle, seed):
    # The default kernel choice (GEMV, skinny, ring by the rounds model, or
    # the register-staged fallback) on random shapes: rows 1..700, widths
    # multiples of 64 with groups 64..256 (odd and even group counts)
    rng = np.random.default_rng(1000 + seed)
    rows = int(rng.choice([1, 3, 17, 64, 65, 200, 333, 700]))
    group = int(rng.choice([64, 128, 256]))
    width = group * int(rng.integers(1, 13))
    columns = int(rng.integers(1, 900))
    x, packed, bits, b = wd.random_case(rng, rows, width, columns, group, bias=bool(seed % 2))
    got = run(x, packed, bits, b, group).astype(np.float64)
    truth = oracle.w4a16_f64(x, packed, bits, group, b)
    assert tolerance.rel_err(got, truth) <= tolerance.FP16_REL_TOL, (rows, width, columns, group)


_SPLIT_CASES = {}


@pytest.mark.parametrize("tile", ["4", "5", "6", "10", "16", "17", "18"])
@pytest.mark.parametrize("splits", ["2", "3", "4"])
@pytest.mark.parametrize("rows,width,columns,group,bias", [(520, 4096, 300, 128, False),
                                                           (300, 2048, 202, 64, True),
                                                           (130, 768, 515, 256, True),
                                                           (65, 128, 33, 64, False)])
def test_split_k_every_ring(oracle, monkeypatch, tile, splits, rows, width, columns, group, bias, knobs):
    # OMNI_W4A16_SPLITS forces split K on a pinned int4 ring: units of
    # (tile, K range), f32 partial sums of the scaled codes, an in-order
    # reduction adding bias. K tile counts 64, 32, 12 and 2 (uneven splits,
    # fewer than asked when a split would be empty), ragged rows and columns,
    # columns % 4 != 0 (the reduction's scalar path); deterministic. One
    # case per shape, its f64 truth computed once.
    knobs.set("OMNI_W4A16_TILE", tile)
    knobs.set("OMNI_W4A16_SPLITS", splits)
    key = (rows, width, columns, group, bias)
    if key not in _SPLIT_CASES:
        rng = np.random.default_rng(rows + width + columns)
        x, packed, bits, b = wd.random_case(rng, rows, width, columns, group, bias=bias)
        _SPLIT_CASES[key] = (x, packed, bits, b, oracle.w4a16_f64(x, packed, bits, group, b))
    x, packed, bits, b, truth = _SPLIT_CASES[key]
    scale = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()
    xd, pd, bd = dev(x), dev(packed), None if b is None else dev(b)
    got = oi.w4a16_linear(xd, pd, scale, bd, group=group)
    again = oi.w4a16_linear(xd, pd, scale, bd, group=group)
    assert tolerance.rel_err(got.cpu().numpy().astype(np.float64), truth) <= tolerance.FP16_REL_TOL, \
        (tile, splits, rows, width, columns)
    assert torch.equal(got, again), "split K must be deterministic"


def test_split_k_workspace_contract(oracle, monkeypatch, knobs):
    # omni_w4a16_gemm_workspace_size reports splits * rows * columns floats
    # for a split shape and 0 otherwise; omni_w4a16_gemm_ws splits less with
    # a smaller workspace, not at all with none, and every result is within
    # the bar.
    from omni_int8 import _lib
    L = _lib.lib()
    knobs.set("OMNI_W4A16_TILE", "4")
    knobs.set("OMNI_W4A16_SPLITS", "4")
    rows, width, columns, group = 300, 4096, 260, 128
    assert L.omni_w4a16_gemm_workspace_size(rows, columns, width, group) == 4 * rows * columns * 4
    assert L.omni_w4a16_gemm_workspace_size(64, columns, width, group) == 0  # skinny route
    assert L.omni_w4a16_gemm_workspace_size(4, columns, width, group) == 0  # GEMV
    assert L.omni_w4a16_gemm_workspace_size(rows, columns, width, 96) == 0  # width % group != 0
    knobs.unset("OMNI_W4A16_TILE")
    knobs.unset("OMNI_W4A16_SPLITS")
    # the launcher's own choice: MiniCPM-V's down projection at M = 1024
    # splits, its K = 3584 linears do not
    assert L.omni_w4a16_gemm_workspace_size(1024, 3584, 18944, 128) >= 2 * 1024 * 3584 * 4
    assert L.omni_w4a16_gemm_workspace_size(1024, 18944, 3584, 128) == 0
    knobs.set("OMNI_W4A16_TILE", "4")
    knobs.set("OMNI_W4A16_SPLITS", "4")
    rng = np.random.default_rng(79)
    x, packed, bits, b = wd.random_case(rng, rows, width, columns, group, bias=True)
    scale = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()
    xd, pd, bd = dev(x), dev(packed), dev(b)
    truth = oracle.w4a16_f64(x, packed, bits, group, b)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for floats in (4 * rows * columns, 2 * rows * columns + 5, 0):
        ws = torch.empty(max(floats, 1) * 4, dtype=torch.uint8, device="cuda")
        out = torch.empty((rows, columns), dtype=torch.float16, device="cuda")
        st = L.omni_w4a16_gemm_ws(xd.data_ptr(), pd.data_ptr(), scale.data_ptr(), group, bd.data_ptr(), rows,
                                  columns, width, out.data_ptr(), ws.data_ptr() if floats else None, floats * 4,
                                  stream)
        assert st == 0, _lib.last_error()
        assert tolerance.rel_err(out.cpu().numpy().astype(np.float64), truth) <= tolerance.FP16_REL_TOL, floats
        outs.append(out)
    knobs.set("OMNI_W4A16_SPLITS", "1")
    plain = oi.w4a16_linear(xd, pd, scale, bd, group=group)
    assert torch.equal(outs[2], plain), "no workspace runs unsplit"
    bad = torch.empty(1024, dtype=torch.uint8, device="cuda")
    st = L.omni_w4a16_gemm_ws(xd.data_ptr(), pd.data_ptr(), scale.data_ptr(), group, bd.data_ptr(), rows, columns,
                              width, outs[0].data_ptr(), bad.data_ptr() + 4, 512, stream)
    assert st == _lib.OMNI_BAD_ARGUMENT


@pytest.mark.parametrize("route", ["0", "1", "2"])
@pytest.mark.parametrize("rows,width,columns,group", [(24, 4096, 8200, 128), (40, 2048, 16400, 64),
                                                      (40, 8192, 4100, 128), (17, 512, 300, 128)])
def test_mid_rows_on_every_route(oracle, monkeypatch, route, rows, width, columns, group, knobs):
    # 17..64 activation rows: the default choice (the first two shapes take
    # the GEMM, the last two the skinny kernel), and each route forced
    knobs.set("OMNI_W8A16_ROUTE", route)
    rng = np.random.default_rng(rows + width + columns + group)
    x, packed, bits, b = wd.random_case(rng, rows, width, columns, group, bias=True)
    got = run(x, packed, bits, b, group).astype(np.float64)
    truth = oracle.w4a16_f64(x, packed, bits, group, b)
    assert tolerance.rel_err(got, truth) <= tolerance.FP16_REL_TOL, (route, rows, width, columns)


@pytest.mark.parametrize("splits", ["auto", "2", "4"])
@pytest.mark.parametrize("rows,width,columns,group,bias", [(16, 4096, 4200, 128, False), (9, 2048, 1000, 64, True),
                                                           (5, 4096, 300, 256, True), (12, 1024, 70, 128, False),
                                                           (16, 3072, 8199, 128, True), (7, 3584, 8300, 128, True),
                                                           (16, 1344, 600, 64, False)])
def test_skinny_split_k(oracle, monkeypatch, splits, rows, width, columns, group, bias, knobs):
    # The int4 split-K skinny kernel (5..16 rows): units of 64 columns x
    # K / splits, partial sums of the scaled codes added in order by the
    # reduction (bias only); forced splits, and the default choice
    # ("auto": K of 3072..4096 over at least 8192 columns), deterministic
    if splits != "auto":
        knobs.set("OMNI_W4A16_SKINNY_SPLIT", splits)
    rng = np.random.default_rng(rows + width + columns + group)
    x, packed, bits, b = wd.random_case(rng, rows, width, columns, group, bias=bias)
    scale = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()
    xd, pd, bd = dev(x), dev(packed), None if b is None else dev(b)
    got = oi.w4a16_linear(xd, pd, scale, bd, group=group)
    again = oi.w4a16_linear(xd, pd, scale, bd, group=group)
    truth = oracle.w4a16_f64(x, packed, bits, group, b)
    assert tolerance.rel_err(got.cpu().numpy().astype(np.float64), truth) <= tolerance.FP16_REL_TOL, \
        (splits, rows, width, columns)
    assert torch.equal(got, again)


def test_skinny_split_k_workspace_size():
    from omni_int8 import _lib
    L = _lib.lib()
    assert L.omni_w4a16_gemm_workspace_size(16, 14336, 4096, 128) == 4 * 16 * 14336 * 4
    assert L.omni_w4a16_gemm_workspace_size(8, 8192, 3072, 128) == 3 * 8 * 8192 * 4
    assert L.omni_w4a16_gemm_workspace_size(16, 4096, 4096, 128) == 0     # one round of workgroups
    assert L.omni_w4a16_gemm_workspace_size(16, 6144, 4096, 128) == 0     # under two rounds
    assert L.omni_w4a16_gemm_workspace_size(16, 18944, 3584, 128) == 4 * 16 * 18944 * 4  # 896-element units
    assert L.omni_w4a16_gemm_workspace_size(16, 8192, 2048, 128) == 0     # K < 3072
    assert L.omni_w4a16_gemm_workspace_size(4, 14336, 4096, 128) == 0     # GEMV
