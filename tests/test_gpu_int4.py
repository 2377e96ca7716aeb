"""INT4 dequantization, GEMV and MFMA GEMM on the GPU vs the CPU oracle.

Bars (from the build's north star): dequantization is bit-exact (one fp32
rounding, as the reference); fp32-output GEMV within relative L2 1e-5 of the
fp64 truth; bf16-output GEMV/GEMM within relative L2 1e-2.
"""
import ctypes
import os

import numpy as np
import pytest

import kc_abi
from kc_abi import ptr, stream
from kc_data import bf16_bits_to_f32, make_int4, normal_bf16, rel_l2

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5
TOL_BF16 = 1e-2


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _dev_bf16(torch, bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


def _host_bf16_bits(t):
    return t.view(__import__("torch").int16).cpu().numpy().view(np.uint16)


def _gemv_f32(torch, packed, scales, zeros, x, rows, cols, gs):
    L = kc_abi.lib()
    dp, ds, dz, dx = (_dev(torch, packed), _dev(torch, scales), _dev(torch, zeros),
                      _dev(torch, x))
    dy = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    print(f"launch_gemv_int4 rows={rows} cols={cols} gs={gs}", flush=True)
    L.launch_gemv_int4(ptr(dp), ptr(ds), ptr(dz), ptr(dx), ptr(dy), rows, cols, gs, stream())
    kc_abi.check("launch_gemv_int4")
    return dy.cpu().numpy()


def _dequant(torch, packed, scales, zeros, rows, cols, gs):
    L = kc_abi.lib()
    dp, ds, dz = _dev(torch, packed), _dev(torch, scales), _dev(torch, zeros)
    out = torch.full((rows, cols), float("nan"), dtype=torch.float32, device="cuda")
    print(f"launch_dequantize_int4 rows={rows} cols={cols} gs={gs}", flush=True)
    L.launch_dequantize_int4(ptr(dp), ptr(ds), ptr(dz), ptr(out), rows, cols, gs, stream())
    kc_abi.check("launch_dequantize_int4")
    return out.cpu().numpy()


def _gemv_bf16(torch, packed, scales, zeros, xb, rows, cols, gs):
    L = kc_abi.lib()
    dp, ds, dz, dx = (_dev(torch, packed), _dev(torch, scales), _dev(torch, zeros),
                      _dev_bf16(torch, xb))
    dy = torch.full((rows,), float("nan"), dtype=torch.bfloat16, device="cuda")
    print(f"kc_gemv_int4_bf16 rows={rows} cols={cols} gs={gs}", flush=True)
    st = L.kc_gemv_int4_bf16(ptr(dp), ptr(ds), ptr(dz), ptr(dx), ptr(dy), rows, cols, gs,
                             stream())
    kc_abi.check("kc_gemv_int4_bf16", st)
    torch.cuda.synchronize()
    return bf16_bits_to_f32(_host_bf16_bits(dy))


# ---------------------------------------------------------------------------
# Reference known-answer tests through the GPU
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["deq_basic", "deq_multigroup", "deq_rng42"])
def test_dequant_reference_kats(gpu, golden, name):
    rows, cols, gs = (int(v) for v in golden[f"{name}_shape"])
    out = _dequant(gpu, golden[f"{name}_packed"], golden[f"{name}_scales"],
                   golden[f"{name}_zeros"], rows, cols, gs)
    np.testing.assert_array_equal(out, golden[f"{name}_expected"])


@pytest.mark.parametrize("name,atol", [("gemv_srand42", 1e-4), ("triton_small", 5e-3),
                                       ("triton_medium", 5e-3), ("triton_gs64", 5e-3)])
def test_gemv_reference_kats(gpu, golden, oracle, name, atol):
    rows, cols, gs = (int(v) for v in golden[f"{name}_shape"])
    packed, scales, zeros = (golden[f"{name}_packed"], golden[f"{name}_scales"],
                             golden[f"{name}_zeros"])
    x = golden[f"{name}_x"]
    y = _gemv_f32(gpu, packed, scales, zeros, x, rows, cols, gs)
    assert np.max(np.abs(y - golden[f"{name}_expected"])) < atol
    truth = oracle.gemv_int4_f64(packed, scales, zeros.reshape(-1), x, rows, cols, gs)
    assert rel_l2(y, truth) < TOL_F32


# ---------------------------------------------------------------------------
# cfg0 and shape coverage (fast and generic paths)
# ---------------------------------------------------------------------------

def test_gemv_cfg0_4096(gpu, oracle):
    """BASELINE cfg0: K = N = 4096, gs 128, fp32 x and y."""
    rows = cols = 4096
    gs = 128
    packed, scales, zeros = make_int4(rows, cols, gs, seed=1)
    x = np.random.default_rng(2).standard_normal(cols).astype(np.float32)
    y = _gemv_f32(gpu, packed, scales, zeros, x, rows, cols, gs)
    zf = zeros.reshape(-1)
    truth = oracle.gemv_int4_f64(packed, scales, zf, x, rows, cols, gs)
    assert rel_l2(y, truth) < TOL_F32
    ref32 = oracle.gemv_int4_refkernel_f32(packed, scales, zf, x, rows, cols, gs)
    assert rel_l2(y, ref32) < 2 * TOL_F32


SHAPES = [
    # (rows, cols, gs): fast path (gs pow2 >= 32)
    (1, 32, 32), (3, 64, 32), (17, 256, 64), (16, 4096, 128), (33, 2080, 32), (3, 36864, 128),
    (64, 14336, 128), (100, 384, 128), (5, 6144, 256), (257, 1024, 1024),
    # generic path: gs < 32, non power of two, tiny K
    (4, 8, 8), (7, 2, 2), (9, 96, 96), (5, 120, 24), (3, 1000, 10), (2, 4, 4),
]


@pytest.mark.parametrize("rows,cols,gs", SHAPES)
def test_gemv_f32_shapes(gpu, oracle, rows, cols, gs):
    packed, scales, zeros = make_int4(rows, cols, gs, seed=rows * 7 + cols)
    x = np.random.default_rng(cols).standard_normal(cols).astype(np.float32)
    y = _gemv_f32(gpu, packed, scales, zeros, x, rows, cols, gs)
    truth = oracle.gemv_int4_f64(packed, scales, zeros.reshape(-1), x, rows, cols, gs)
    assert rel_l2(y, truth) < TOL_F32


# Staged-kernel variants: 4 rows per wave (K = 4096 from N = 4096, K = 8192
# from N = 8192; ragged N, 16- and 64-lane slot maps) and x beyond 64 KB of
# LDS (fp32 x at K > 15872, up to the 160 KB of K = 32768).
# Below N = 8192 with K = 2048 x 2..8 the fp32 GEMV takes the per-lane-x
# kernel instead (ragged N, groups 32..256).
F32_STAGED_SHAPES = [(8192, 4096, 32), (8195, 4096, 64), (8192, 8192, 128), (8200, 8192, 32),
                     (8200, 16384, 128), (33, 20480, 64), (9, 32768, 128), (5, 31744, 32),
                     (4096, 4096, 32), (4099, 4096, 64), (8191, 4096, 128), (100, 6144, 64),
                     (4097, 14336, 128), (17, 8192, 256), (40, 16384, 128)]


@pytest.mark.parametrize("rows,cols,gs", F32_STAGED_SHAPES)
def test_gemv_f32_staged_variants(gpu, oracle, rows, cols, gs):
    packed, scales, zeros = make_int4(rows, cols, gs, seed=rows * 5 + cols)
    x = np.random.default_rng(cols + 1).standard_normal(cols).astype(np.float32)
    y = _gemv_f32(gpu, packed, scales, zeros, x, rows, cols, gs)
    truth = oracle.gemv_int4_f64(packed, scales, zeros.reshape(-1), x, rows, cols, gs)
    assert rel_l2(y, truth) < TOL_F32


@pytest.mark.parametrize("rows,cols,gs", SHAPES)
def test_dequant_shapes_bit_exact(gpu, oracle, rows, cols, gs):
    packed, scales, zeros = make_int4(rows, cols, gs, seed=rows * 3 + cols)
    out = _dequant(gpu, packed, scales, zeros, rows, cols, gs)
    exp = oracle.dequantize_int4(packed, scales, zeros.reshape(-1), rows, cols, gs)
    np.testing.assert_array_equal(out, exp)


def test_gemv_sign_and_zero_point_invariants(gpu):
    rows, cols, gs = 64, 1024, 128
    x = np.random.default_rng(3).standard_normal(cols).astype(np.float32)
    G = cols // gs
    # 0x33 with zero point 3 -> all weights 0 -> y == 0.  The fast path folds
    # the zero point per 32-k chunk as s*(sum n'x - (8+z) sum x), so the two
    # sums cancel to within fp32 rounding of s * 11 * sum|x| rather than to 0.
    y = _gemv_f32(gpu, np.full((rows, cols // 2), 0x33, np.uint8),
                  np.full((rows, G), 0.01, np.float32), np.full((rows, G // 2), 0x33, np.uint8),
                  x, rows, cols, gs)
    scale = 0.01 * 11 * np.abs(x).sum()
    assert np.all(np.abs(y) <= 1e-6 * scale)
    # 0x88 with zero point 8 -> every weight -16 * s (sign extension)
    y = _gemv_f32(gpu, np.full((rows, cols // 2), 0x88, np.uint8),
                  np.full((rows, G), 0.5, np.float32), np.full((rows, G // 2), 0x88, np.uint8),
                  x, rows, cols, gs)
    np.testing.assert_allclose(y, np.full(rows, -8.0 * x.astype(np.float64).sum()), rtol=1e-5)


def test_gemv_linearity(gpu):
    rows, cols, gs = 256, 4096, 128
    packed, scales, zeros = make_int4(rows, cols, gs, seed=4)
    rng = np.random.default_rng(5)
    x1 = rng.standard_normal(cols).astype(np.float32)
    x2 = rng.standard_normal(cols).astype(np.float32)
    y1 = _gemv_f32(gpu, packed, scales, zeros, x1, rows, cols, gs)
    y2 = _gemv_f32(gpu, packed, scales, zeros, x2, rows, cols, gs)
    y3 = _gemv_f32(gpu, packed, scales, zeros, (2 * x1 - x2).astype(np.float32), rows, cols, gs)
    assert rel_l2(y3, 2 * y1.astype(np.float64) - y2) < 1e-5
    y0 = _gemv_f32(gpu, packed, scales, zeros, np.zeros(cols, np.float32), rows, cols, gs)
    assert np.all(y0 == 0.0)


def test_gemv_unaligned_pointers_take_generic_path(gpu, oracle):
    torch = gpu
    rows, cols, gs = 8, 512, 128
    packed, scales, zeros = make_int4(rows, cols, gs, seed=6)
    x = np.random.default_rng(7).standard_normal(cols + 1).astype(np.float32)
    L = kc_abi.lib()
    dp = torch.empty(packed.size + 3, dtype=torch.uint8, device="cuda")
    dp[3:] = _dev(torch, packed.reshape(-1))
    dx = _dev(torch, x)
    ds, dz = _dev(torch, scales), _dev(torch, zeros)
    dy = torch.empty(rows, dtype=torch.float32, device="cuda")
    L.launch_gemv_int4(ctypes.c_void_p(dp.data_ptr() + 3), ptr(ds), ptr(dz),
                       ctypes.c_void_p(dx.data_ptr() + 4), ptr(dy), rows, cols, gs, stream())
    kc_abi.check("launch_gemv_int4")
    truth = oracle.gemv_int4_f64(packed, scales, zeros.reshape(-1), x[1:], rows, cols, gs)
    assert rel_l2(dy.cpu().numpy(), truth) < TOL_F32


def test_reference_launchers_empty_shapes(gpu):
    L = kc_abi.lib()
    L.kc_get_last_error()
    L.launch_gemv_int4(None, None, None, None, None, 0, 256, 128, stream())
    L.launch_dequantize_int4(None, None, None, None, 0, 256, 128, stream())
    assert L.kc_get_last_error() == 0


# ---------------------------------------------------------------------------
# bf16 GEMV at the Llama-3-8B decode shapes (BASELINE cfg2)
# ---------------------------------------------------------------------------

LLAMA_SHAPES = [(6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336)]  # (N, K)


@pytest.mark.parametrize("rows,cols", LLAMA_SHAPES)
def test_gemv_bf16_llama_shapes(gpu, oracle, rows, cols):
    gs = 128
    packed, scales, zeros = make_int4(rows, cols, gs, seed=2000 + rows + cols)
    xb = normal_bf16(cols, seed=2001 + cols)
    y = _gemv_bf16(gpu, packed, scales, zeros, xb, rows, cols, gs)
    truth = oracle.gemv_int4_f64(packed, scales, zeros.reshape(-1), bf16_bits_to_f32(xb),
                                 rows, cols, gs)
    assert rel_l2(y, truth) < TOL_BF16
    # tighter: bf16 output rounding alone is ~1e-3
    assert rel_l2(y, truth) < 3e-3


@pytest.mark.parametrize("rows,cols,gs", [(5, 96, 32), (3, 100, 10), (70, 2048, 64),
                                           # K = 2048 x KW, x per lane: 4 or 8 rows per
                                           # wave, ragged row counts, groups 32..256
                                           (1000, 8192, 128), (20000, 6144, 64),
                                           (17, 16384, 256), (4099, 10240, 32),
                                           (16384, 4096, 128), (16385, 4096, 128),
                                           (100, 8192, 512), (9, 4096, 2048),
                                           (20480, 4096, 32), (16392, 4096, 256)])
def test_gemv_bf16_other_shapes(gpu, oracle, rows, cols, gs):
    packed, scales, zeros = make_int4(rows, cols, gs, seed=rows + cols)
    xb = normal_bf16(cols, seed=cols)
    y = _gemv_bf16(gpu, packed, scales, zeros, xb, rows, cols, gs)
    truth = oracle.gemv_int4_f64(packed, scales, zeros.reshape(-1), bf16_bits_to_f32(xb),
                                 rows, cols, gs)
    assert rel_l2(y, truth) < 3e-3


# ---------------------------------------------------------------------------
# MFMA small-batch GEMM (BASELINE cfg3) vs the reference GEMV per row
# ---------------------------------------------------------------------------

def _gemm(torch, packed, scales, zeros, xb, m, rows, cols, gs):
    L = kc_abi.lib()
    dp, ds, dz, dx = (_dev(torch, packed), _dev(torch, scales), _dev(torch, zeros),
                      _dev_bf16(torch, xb))
    dy = torch.full((m, rows), float("nan"), dtype=torch.bfloat16, device="cuda")
    print(f"kc_gemm_int4_bf16 m={m} rows={rows} cols={cols} gs={gs}", flush=True)
    st = L.kc_gemm_int4_bf16(ptr(dp), ptr(ds), ptr(dz), ptr(dx), ptr(dy), m, rows, cols, gs,
                             stream())
    kc_abi.check("kc_gemm_int4_bf16", st)
    torch.cuda.synchronize()
    return bf16_bits_to_f32(_host_bf16_bits(dy)).reshape(m, rows), (dp, ds, dz, dx)


@pytest.mark.parametrize("m", [4, 16, 32, 64])
def test_gemm_cfg3(gpu, oracle, m):
    """M in {4, 16, 64}, K = 8192, N = 28672, gs 128.  Every output row against
    the fp64 oracle (the reference GEMV per activation row, its rows split over
    the host's cores): relative L2 per activation row and over the whole Y;
    every row also against an fp32 GPU reference built from the bit-exact
    dequantization."""
    torch = gpu
    rows, cols, gs = 28672, 8192, 128
    packed, scales, zeros = make_int4(rows, cols, gs, seed=3000 + m)
    xb = normal_bf16((m, cols), seed=3001 + m)
    y, (dp, ds, dz, dx) = _gemm(torch, packed, scales, zeros, xb, m, rows, cols, gs)
    threads = min(16, len(os.sched_getaffinity(0)))
    print(f"cfg3 m={m}: fp64 oracle over {rows} rows on {threads} threads", flush=True)
    truth = oracle.gemm_int4_bf16_f64(packed, scales, zeros.reshape(-1), xb, m, rows, cols, gs,
                                      threads=threads)
    assert np.all(np.isfinite(y))
    assert rel_l2(y, truth) < 3e-3
    for i in range(m):
        assert rel_l2(y[i], truth[i]) < 3e-3, i
    L = kc_abi.lib()
    W = torch.empty(rows, cols, dtype=torch.float32, device="cuda")
    L.launch_dequantize_int4(ptr(dp), ptr(ds), ptr(dz), ptr(W), rows, cols, gs, stream())
    kc_abi.check("launch_dequantize_int4")
    ref = (dx.float() @ W.t()).cpu().numpy()
    assert rel_l2(y, ref) < 3e-3


@pytest.mark.parametrize("m,rows,cols,gs", [(1, 100, 1024, 128), (3, 64, 256, 128),
                                            (17, 130, 2048, 256), (33, 48, 640, 128),
                                            (64, 16, 128, 128), (5, 40, 512, 64),
                                            # M <= 4, X resident in LDS: ragged row
                                            # tiles, spare waves, odd T-block counts,
                                            # larger groups
                                            (2, 250, 384, 128), (1, 17, 128, 128),
                                            (4, 1000, 1280, 256), (3, 4096, 4096, 128),
                                            (4, 7 * 16 * 3 + 5, 2048, 512),
                                            # M <= 4 whose X does not fit in LDS
                                            (4, 33, 32768, 128),
                                            # M 5..8: X in LDS in one, two and four
                                            # phases of K; M 9..16 on the K-split
                                            # kernel, or past its LDS on the chunked one
                                            (16, 48, 1024, 128), (8, 300, 4096, 128),
                                            (12, 257, 2048, 256), (16, 100, 8192, 128),
                                            (6, 7 * 16 + 1, 8192, 512), (8, 500, 8192, 128),
                                            (12, 100, 24576, 128), (9, 40, 2048, 256),
                                            # M 17..64, K split over four waves:
                                            # ragged rows and activation tiles,
                                            # waves with no T-block (K < 512),
                                            # ranges of unequal length
                                            (33, 70, 1024, 128), (64, 7 * 16 * 2 + 9, 2048, 256),
                                            (48, 200, 8192, 128), (20, 224, 4096, 128),
                                            (32, 1000, 4096, 128), (40, 113, 16384, 128),
                                            (17, 7, 256, 256), (63, 1, 512, 128),
                                            (26, 130, 1152, 128), (40, 200, 4096, 512),
                                            # M 33..64 whose coefficients do not fit
                                            # in LDS: the X-resident fallback
                                            (64, 50, 24576, 128),
                                            # reference layout in pairs of T-blocks:
                                            # one pair per wave, three and five pairs
                                            # with groups of 256 / 512, ragged rows, and
                                            # K at the pair form's LDS limit for one to
                                            # four activation tiles; three pairs with a
                                            # last group of two T-blocks for the
                                            # zero-point pass
                                            (3, 200, 1024, 128), (2, 77, 3072, 256),
                                            (5, 1000, 5120, 512), (8, 130, 12288, 128),
                                            (32, 100, 9216, 128), (20, 60, 10240, 128),
                                            (36, 90, 12288, 128), (64, 100, 8192, 128),
                                            (50, 77, 3072, 256),
                                            # four activation tiles, one T-block at a
                                            # time: tiles past the last row, two
                                            # T-blocks per wave, K at the pair form's
                                            # limit for one tile fewer
                                            (50, 80, 3072, 256), (49, 224, 1024, 128),
                                            (64, 96, 8192, 128),
                                            # the pair form with fewer rows than one
                                            # 16-row tile (every row clamped to N - 1)
                                            (9, 5, 2048, 128), (2, 1, 1024, 128),
                                            # M 33..64 with fewer rows than a workgroup's
                                            # 112, K 2048-6144
                                            (40, 40, 2048, 128), (64, 16, 4096, 128),
                                            (35, 200, 6144, 128), (57, 1000, 2048, 128)])
def test_gemm_shapes(gpu, oracle, m, rows, cols, gs):
    packed, scales, zeros = make_int4(rows, cols, gs, seed=m * 1000 + rows)
    xb = normal_bf16((m, cols), seed=m + rows)
    y, _ = _gemm(gpu, packed, scales, zeros, xb, m, rows, cols, gs)
    truth = oracle.gemm_int4_bf16_f64(packed, scales, zeros.reshape(-1), xb, m, rows, cols, gs)
    assert rel_l2(y, truth) < 3e-3


# ---------------------------------------------------------------------------
# A decode step's GEMVs in one launch (kc_gemv_int4_bf16_chain)
# ---------------------------------------------------------------------------

def _run_chain(torch, specs, wire, seed=3000):
    """specs: (rows, cols, gs) per op; wire[i] = j takes op i's x from the
    first cols entries of op j's y (j < i), -1 a fresh random x.  Runs the
    chain and returns, per op, its weights, the x it read and its y."""
    import kernel_craft_torch_ops as ops
    dev_ops, weights, ys = [], [], []
    for i, (rows, cols, gs) in enumerate(specs):
        packed, scales, zeros = make_int4(rows, cols, gs, seed=seed + 7 * i + rows + cols)
        if wire[i] < 0:
            x = _dev_bf16(torch, normal_bf16(cols, seed=seed + 100 + i))
        else:
            x = ys[wire[i]][:cols]
            assert x.numel() == cols, "an op's x must fit in the earlier op's y"
        y = torch.full((rows,), float("nan"), dtype=torch.bfloat16, device="cuda")
        ys.append(y)
        dev_ops.append((_dev(torch, packed), _dev(torch, scales), _dev(torch, zeros), x, y,
                        rows, cols, gs))
        weights.append((packed, scales, zeros))
    print(f"chain specs={specs} wire={wire}", flush=True)
    ops.int4_gemv_bf16_chain(dev_ops)
    torch.cuda.synchronize()
    return [(w, _host_bf16_bits(d[3]), bf16_bits_to_f32(_host_bf16_bits(d[4])))
            for w, d in zip(weights, dev_ops)]


def _check_chain(oracle, specs, results, tol=3e-3):
    for (rows, cols, gs), ((packed, scales, zeros), xb, y) in zip(specs, results):
        truth = oracle.gemv_int4_f64(packed, scales, zeros.reshape(-1), bf16_bits_to_f32(xb),
                                     rows, cols, gs)
        assert np.all(np.isfinite(y)), (rows, cols, gs)
        assert rel_l2(y, truth) < tol, (rows, cols, gs, rel_l2(y, truth))


def test_chain_llama_decode_layer(gpu, oracle):
    """QKV -> O -> gate/up -> down from one call, each op reading the previous
    op's output."""
    specs = [(6144, 4096, 128), (4096, 4096, 128), (28672, 4096, 128), (4096, 14336, 128)]
    _check_chain(oracle, specs, _run_chain(gpu, specs, [-1, 0, 1, 2]))


# the standalone kernel's chunks-per-lane counts 1..8 and group sizes 128..4096
CHAIN_SHAPES = [(13001, 2048, 128), (3, 128, 128), (12288, 4096, 256), (50, 4096, 128),
                (6150, 6144, 128), (6200, 8192, 512), (777, 10240, 128), (300, 12288, 1024),
                (4096, 14336, 128), (9, 16384, 128), (64, 4096, 4096)]


@pytest.mark.parametrize("rows,cols,gs", CHAIN_SHAPES)
def test_chain_shapes(gpu, oracle, rows, cols, gs):
    specs = [(rows, cols, gs)]
    _check_chain(oracle, specs, _run_chain(gpu, specs, [-1], seed=rows + cols))


def test_chain_eight_ops_in_a_line(gpu, oracle):
    specs = [(2048, 1024, 128), (4096, 2048, 128), (1024, 4096, 256), (8192, 1024, 128),
             (512, 8192, 128), (3000, 512, 128), (640, 3000 - 3000 % 128, 128), (100, 640, 128)]
    wire = [-1, 0, 1, 2, 3, 4, 5, 6]
    _check_chain(oracle, specs, _run_chain(gpu, specs, wire, seed=77))


def test_chain_other_group_sizes_and_long_rows(gpu, oracle):
    """Group size 64 and cols above 16384 (the generic and wide GEMV routes)."""
    specs = [(300, 2048, 64), (500, 16512, 128), (200, 256, 128)]
    _check_chain(oracle, specs, _run_chain(gpu, specs, [-1, -1, 0], seed=5))


def test_chain_argument_errors(gpu):
    import kernel_craft_torch_ops as ops
    L = kc_abi.lib()
    arr = (ops.GemvOp * 9)()
    assert L.kc_gemv_int4_bf16_chain(ctypes.cast(arr, ctypes.c_void_p), 9, stream()) == 1
    assert L.kc_gemv_int4_bf16_chain(None, 1, stream()) == 1
    arr[0].rows, arr[0].cols, arr[0].group_size = 4, 256, 100
    assert L.kc_gemv_int4_bf16_chain(ctypes.cast(arr, ctypes.c_void_p), 1, stream()) == 1
    arr[0].group_size = 128
    assert L.kc_gemv_int4_bf16_chain(ctypes.cast(arr, ctypes.c_void_p), 1, stream()) == 1  # nulls
    assert L.kc_gemv_int4_bf16_chain(None, 0, stream()) == 0
    L.kc_get_last_error()


# ---------------------------------------------------------------------------
# Runs of independent ops: one launch of the fused tile
# ---------------------------------------------------------------------------

def _fused_tile_takes(rows, cols, gs):
    return cols % 2048 == 0 and 2 <= cols // 2048 <= 8 and gs >= 32 and gs & (gs - 1) == 0


def _same_as_standalone(rows, cols, gs):
    """kc_gemv_int4_bf16 takes the per-lane-x kernel, whose per-row
    arithmetic the fused tile repeats: the outputs are equal bit for bit
    (at K = 4096 with N > 16384 it takes the LDS-staged kernel, which sums
    in another order)."""
    return _fused_tile_takes(rows, cols, gs) and not (cols == 4096 and rows > 16384)


def _check_run(torch, oracle, specs, results, tol=3e-3):
    _check_chain(oracle, specs, results, tol)
    for (rows, cols, gs), ((packed, scales, zeros), xb, y) in zip(specs, results):
        if _same_as_standalone(rows, cols, gs):
            alone = _gemv_bf16(torch, packed, scales, zeros, xb, rows, cols, gs)
            np.testing.assert_array_equal(y.view(np.uint32), alone.view(np.uint32),
                                          err_msg=str((rows, cols, gs)))


FUSED_RUNS = [
    # the decode layer with independent inputs (the bench's step): one launch
    [(6144, 4096, 128), (4096, 4096, 128), (28672, 4096, 128), (4096, 14336, 128)],
    # every KW, ragged row counts (tiles of 16, 8, 8, 4, 4, 4, 4 rows)
    [(100, 4096, 128), (37, 6144, 64), (1000, 8192, 32), (5, 10240, 256), (333, 12288, 128),
     (17, 14336, 128), (64, 16384, 512)],
    # group sizes 32 .. 2048 at K = 4096, and single rows
    [(17, 4096, 32), (33, 4096, 64), (65, 4096, 2048), (1, 4096, 128), (1, 14336, 128)],
    # the fused tile next to ops it does not take (K = 2048, K not 2048 KW,
    # K above 16384): those launch on their own, the neighbours keep theirs
    [(100, 4096, 128), (50, 2048, 128), (60, 8192, 128), (70, 8192 + 2048, 128),
     (40, 5120, 128), (30, 18432, 128), (20, 4096, 128), (10, 6144, 128)],
    # runs of up to four ops (weight pointers passed in preloaded arguments):
    # full and ragged last tiles side by side, and three ops
    [(48, 4096, 128), (37, 6144, 64), (1000, 8192, 32), (5, 14336, 128)],
    [(4100, 10240, 128), (16, 4096, 256), (9, 12288, 128)],
]


@pytest.mark.parametrize("specs", FUSED_RUNS, ids=["decode_layer", "every_kw", "group_sizes", "mixed",
                                                   "four_ragged", "three"])
def test_chain_fused_run(gpu, oracle, specs):
    results = _run_chain(gpu, specs, [-1] * len(specs), seed=4000 + len(specs))
    _check_run(gpu, oracle, specs, results)


def test_chain_runs_cut_at_dependencies(gpu, oracle):
    """A, B independent; C reads A's y; D independent of C (but after it):
    the runs are [A, B] and [C, D].  Every op matches its stand-alone GEMV on
    the x it read."""
    specs = [(4096, 4096, 128), (300, 8192, 128), (500, 4096, 128), (200, 14336, 128)]
    _check_run(gpu, oracle, specs, _run_chain(gpu, specs, [-1, -1, 0, -1], seed=4100))


def test_chain_write_after_read_is_ordered(gpu, oracle):
    """Op B overwrites the buffer op A reads its x from: B must run after A
    (another run), so A sees the original x."""
    import kernel_craft_torch_ops as ops
    torch = gpu
    buf = _dev_bf16(torch, normal_bf16(8192, seed=4200))
    x_orig = _host_bf16_bits(buf[:4096].clone())
    pa, sa, za = make_int4(256, 4096, 128, seed=4201)
    pb, sb, zb = make_int4(8192, 4096, 128, seed=4202)
    xb_bits = normal_bf16(4096, seed=4203)
    ya = torch.empty(256, dtype=torch.bfloat16, device="cuda")
    chain = [(_dev(torch, pa), _dev(torch, sa), _dev(torch, za), buf[:4096], ya, 256, 4096, 128),
             (_dev(torch, pb), _dev(torch, sb), _dev(torch, zb), _dev_bf16(torch, xb_bits), buf,
              8192, 4096, 128)]
    print("chain write-after-read", flush=True)
    ops.int4_gemv_bf16_chain(chain)
    torch.cuda.synchronize()
    got_a = bf16_bits_to_f32(_host_bf16_bits(ya))
    np.testing.assert_array_equal(got_a.view(np.uint32),
                                  _gemv_bf16(torch, pa, sa, za, x_orig, 256, 4096, 128).view(np.uint32))
    got_b = bf16_bits_to_f32(_host_bf16_bits(buf))
    np.testing.assert_array_equal(got_b.view(np.uint32),
                                  _gemv_bf16(torch, pb, sb, zb, xb_bits, 8192, 4096, 128).view(np.uint32))


def test_chain_zero_row_ops_inside_a_run(gpu, oracle):
    """Ops with rows == 0 are skipped; the ops around them still form one run."""
    import kernel_craft_torch_ops as ops
    torch = gpu
    specs = [(64, 4096, 128), (0, 4096, 128), (48, 8192, 128), (0, 14336, 128), (32, 14336, 128)]
    chain, host = [], []
    for i, (rows, cols, gs) in enumerate(specs):
        p, s, z = make_int4(max(rows, 1), cols, gs, seed=4300 + i)
        xbits = normal_bf16(cols, seed=4310 + i)
        y = torch.full((max(rows, 1),), 7.0, dtype=torch.bfloat16, device="cuda")
        chain.append((_dev(torch, p), _dev(torch, s), _dev(torch, z), _dev_bf16(torch, xbits), y,
                      rows, cols, gs))
        host.append((p, s, z, xbits))
    print("chain with zero-row ops", flush=True)
    ops.int4_gemv_bf16_chain(chain)
    torch.cuda.synchronize()
    for (rows, cols, gs), (p, s, z, xbits), d in zip(specs, host, chain):
        got = bf16_bits_to_f32(_host_bf16_bits(d[4]))
        if rows == 0:
            assert np.all(got == 7.0), "an op with no rows writes nothing"
            continue
        np.testing.assert_array_equal(got.view(np.uint32),
                                      _gemv_bf16(torch, p, s, z, xbits, rows, cols, gs).view(np.uint32))


def test_chain_fused_run_graph_replays(gpu, oracle):
    """A fused run (the decode layer with independent inputs) captured in a
    HIP graph: every replay equals the eager call bit for bit, with eager
    work on the same buffers between replays."""
    import kernel_craft_torch_ops as ops
    torch = gpu
    specs = FUSED_RUNS[0]
    chain = []
    for i, (rows, cols, gs) in enumerate(specs):
        p, s, z = make_int4(rows, cols, gs, seed=4400 + i)
        chain.append((_dev(torch, p), _dev(torch, s), _dev(torch, z),
                      _dev_bf16(torch, normal_bf16(cols, seed=4410 + i)),
                      torch.empty(rows, dtype=torch.bfloat16, device="cuda"), rows, cols, gs))
    print("fused run: eager", flush=True)
    ops.int4_gemv_bf16_chain(chain)
    torch.cuda.synchronize()
    eager = [d[4].clone() for d in chain]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    print("fused run: capture", flush=True)
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            ops.int4_gemv_bf16_chain(chain)
    torch.cuda.current_stream().wait_stream(side)
    for rep in range(3):
        for d in chain:
            d[4].fill_(3.0)
        torch.cuda.synchronize()
        print(f"fused run: replay {rep}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        for d, e in zip(chain, eager):
            assert torch.equal(d[4].view(torch.int16), e.view(torch.int16)), rep
