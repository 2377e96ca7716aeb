"""RMSNorm and the fused RMSNorm -> INT4 GEMV on the GPU vs the CPU oracle.

Bars: launch_rmsnorm and kc_rmsnorm_bf16 bit for bit against the oracle's
fixed-order restatement (kco_rmsnorm_*_lanes: the library's summation order,
with FMA), and within the reference tests' own max-abs bars (1e-5 for rows
of 8 and 64 values, 1e-4 beyond; tests/test_mamba_ops.cpp:219-300,
test_mamba_bindings.py:251-300) of the oracle of the reference's CPU check,
which sums in index order.  The fused RMSNorm -> FP8 quantizer bit for bit
against the oracle composition (fixed-order RMSNorm, then the per-token
quantizer on its bf16 output) and against the two library launches.  The fused
GEMV's bf16 output is held to relative L2 3e-3 of the fp64 GEMV of its own
bf16 input (bf16(gamma h), scaled by rms_inv), and to the bf16 bar, 1e-2,
of the unrounded fp64 composition.
"""
import numpy as np
import pytest

import kc_abi
from kc_abi import ptr, stream
from kc_data import bf16_bits_to_f32, f32_to_bf16_bits, make_int4, normal_bf16, rel_l2

pytestmark = pytest.mark.gpu


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _dev_bf16(torch, bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


def _bits(t):
    return t.view(__import__("torch").int16).cpu().numpy().view(np.uint16)


def _rmsnorm_f32(torch, x, g, eps=1e-6, offset=0):
    """launch_rmsnorm; offset (in floats) moves every pointer off 16-byte
    alignment to take the scalar path."""
    L = kc_abi.lib()
    rows, D = x.shape
    bx = torch.zeros(x.size + offset, dtype=torch.float32, device="cuda")
    bg = torch.zeros(D + offset, dtype=torch.float32, device="cuda")
    by = torch.full((x.size + offset,), float("nan"), dtype=torch.float32, device="cuda")
    bx[offset:] = _dev(torch, x.reshape(-1))
    bg[offset:] = _dev(torch, g)
    print(f"launch_rmsnorm rows={rows} D={D} offset={offset}", flush=True)
    L.launch_rmsnorm(ptr(bx[offset:]), ptr(bg[offset:]), ptr(by[offset:]), rows, D, eps, stream())
    torch.cuda.synchronize()
    kc_abi.check("launch_rmsnorm")
    return by[offset:].cpu().numpy().reshape(rows, D)


@pytest.mark.parametrize("name,tol", [("rms_basic", 1e-5), ("rms_d768", 1e-4), ("rms_d4096", 1e-4),
                                      ("rms_py_rng3", 1e-5)])
def test_rmsnorm_reference_kats(gpu, golden, name, tol):
    x, g = golden[f"{name}_x"], golden[f"{name}_g"]
    y = _rmsnorm_f32(gpu, x, g)
    assert np.max(np.abs(y - golden[f"{name}_expected"])) < tol


@pytest.mark.parametrize("rows,D,offset", [(1, 4096, 0), (37, 4096, 0), (5, 256, 0), (3, 64, 0),
                                           (9, 8192, 0), (2, 12, 0), (4, 777, 0), (6, 1024, 1),
                                           (3, 20000, 0), (0, 64, 0)])
def test_rmsnorm_f32_shapes(gpu, oracle, rows, D, offset):
    rng = np.random.default_rng(rows * 31 + D)
    x = rng.uniform(-2, 2, (rows, D)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, D).astype(np.float32)
    y = _rmsnorm_f32(gpu, x, g, 1e-6, offset)
    if rows:
        np.testing.assert_array_equal(y, oracle.rmsnorm_lanes(x, g, 1e-6))
        exp = oracle.rmsnorm(x, g, 1e-6)
        assert np.max(np.abs(y - exp)) <= 2e-5 * np.max(np.abs(exp))


def test_rmsnorm_unit_and_constant_rows(gpu):
    """test_mamba_bindings.py:288-310: a constant row gives g; with g = 1 the
    output's rms is 1."""
    y = _rmsnorm_f32(gpu, np.full((4, 64), 2.0, np.float32), np.ones(64, np.float32))
    assert np.max(np.abs(y - 1.0)) < 1e-5
    x = np.random.default_rng(22).uniform(-1, 1, (32, 256)).astype(np.float32)
    y = _rmsnorm_f32(gpu, x, np.ones(256, np.float32))
    assert np.max(np.abs(np.sqrt(np.mean(y.astype(np.float64) ** 2, axis=1)) - 1.0)) < 1e-4


@pytest.mark.parametrize("rows,D", [(1, 4096), (16, 4096), (7, 8192), (3, 14336), (5, 100),
                                    (4, 20000)])
def test_rmsnorm_bf16(gpu, oracle, rows, D):
    L = kc_abi.lib()
    rng = np.random.default_rng(D + rows)
    xb = f32_to_bf16_bits(rng.standard_normal((rows, D)).astype(np.float32) * 3)
    gb = f32_to_bf16_bits(rng.uniform(0.5, 1.5, D).astype(np.float32))
    dx, dg = _dev_bf16(gpu, xb), _dev_bf16(gpu, gb)
    dy = gpu.empty(rows, D, dtype=gpu.bfloat16, device="cuda")
    print(f"kc_rmsnorm_bf16 rows={rows} D={D}", flush=True)
    st = L.kc_rmsnorm_bf16(ptr(dx), ptr(dg), ptr(dy), rows, D, 1e-5, stream())
    kc_abi.check("kc_rmsnorm_bf16", st)
    gpu.cuda.synchronize()
    np.testing.assert_array_equal(_bits(dy), oracle.rmsnorm_lanes(xb, gb, 1e-5))
    got = bf16_bits_to_f32(_bits(dy))
    exp = bf16_bits_to_f32(oracle.rmsnorm(xb, gb, 1e-5))
    ulp = np.abs(exp) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - exp) <= ulp)
    assert np.mean(got == exp) > 0.99


def _fused(torch, packed, scales, zeros, hb, gb, rows, cols, gs, eps=1e-5, gamma_offset=0):
    L = kc_abi.lib()
    dp, ds, dz = _dev(torch, packed), _dev(torch, scales), _dev(torch, zeros)
    dh = _dev_bf16(torch, hb)
    gbuf = torch.zeros(cols + gamma_offset, dtype=torch.bfloat16, device="cuda")
    gbuf[gamma_offset:] = _dev_bf16(torch, gb)
    dy = torch.full((rows,), float("nan"), dtype=torch.bfloat16, device="cuda")
    print(f"kc_rmsnorm_gemv_int4_bf16 rows={rows} cols={cols} gs={gs} goff={gamma_offset}",
          flush=True)
    st = L.kc_rmsnorm_gemv_int4_bf16(ptr(dh), ptr(gbuf[gamma_offset:]), eps, ptr(dp), ptr(ds),
                                     ptr(dz), ptr(dy), rows, cols, gs, stream())
    kc_abi.check("kc_rmsnorm_gemv_int4_bf16", st)
    torch.cuda.synchronize()
    return bf16_bits_to_f32(_bits(dy)), (dp, ds, dz, dh)


@pytest.mark.parametrize("rows,cols,gs,goff", [(6144, 4096, 128, 0), (512, 14336, 128, 0),
                                               (20000, 8192, 128, 0), (28672, 4096, 128, 0),
                                               (17000, 4096, 32, 0),
                                               (300, 20480, 128, 0), (77, 1024, 64, 0),
                                               (33, 2080, 32, 0), (40, 384, 128, 1),
                                               (16, 96, 24, 0)])
def test_rmsnorm_gemv_fused(gpu, oracle, rows, cols, gs, goff):
    """The per-lane-x kernel (K = 2048 x 2..8), the LDS-staged kernel (gate/up,
    K 20480, small K), and the generic path (unaligned gamma, groups that are
    not a power of two)."""
    packed, scales, zeros = make_int4(rows, cols, gs, seed=rows + cols)
    rng = np.random.default_rng(cols)
    hb = f32_to_bf16_bits(rng.standard_normal(cols).astype(np.float32) * 4)
    gb = f32_to_bf16_bits(rng.uniform(0.5, 1.5, cols).astype(np.float32))
    y, _ = _fused(gpu, packed, scales, zeros, hb, gb, rows, cols, gs, 1e-5, goff)
    # y = rms_inv * W bf16(gamma h), the GEMV from the fp64 oracle
    h = bf16_bits_to_f32(hb)
    rinv = 1.0 / np.sqrt(np.mean(h.astype(np.float64) ** 2) + 1e-5)
    xg = bf16_bits_to_f32(f32_to_bf16_bits(bf16_bits_to_f32(gb) * h))
    truth = oracle.gemv_int4_f64(packed, scales, zeros.reshape(-1), xg, rows, cols, gs) * rinv
    assert rel_l2(y, truth) < 3e-3
    # against the unrounded composition (the reference's fp32 RMSNorm feeding
    # its fp32 GEMV), the bf16 bar: where x is rounded moves y by up to about
    # 1e-2 here, because these weights' common offset (-8 - z) makes the row
    # sums small against sum |w x|
    exact = oracle.gemv_int4_f64(packed, scales, zeros.reshape(-1),
                                 bf16_bits_to_f32(gb).astype(np.float64) * h * rinv, rows, cols, gs)
    assert rel_l2(y, exact) < 1e-2


def test_rmsnorm_gemv_fused_matches_two_launches(gpu, oracle):
    """The fused launch and kc_rmsnorm_bf16 followed by kc_gemv_int4_bf16
    (Llama gate/up shape) round x to bf16 at different places (before and
    after the normalization); both meet the bf16 bar against the unrounded
    fp64 composition."""
    L = kc_abi.lib()
    rows, cols, gs = 28672, 4096, 128
    packed, scales, zeros = make_int4(rows, cols, gs, seed=8)
    rng = np.random.default_rng(9)
    hb = f32_to_bf16_bits(rng.standard_normal(cols).astype(np.float32))
    gb = f32_to_bf16_bits(rng.uniform(0.5, 1.5, cols).astype(np.float32))
    y, (dp, ds, dz, dh) = _fused(gpu, packed, scales, zeros, hb, gb, rows, cols, gs)
    dg = _dev_bf16(gpu, gb)
    dx = gpu.empty(cols, dtype=gpu.bfloat16, device="cuda")
    dy = gpu.empty(rows, dtype=gpu.bfloat16, device="cuda")
    print("kc_rmsnorm_bf16 + kc_gemv_int4_bf16 gate/up", flush=True)
    kc_abi.check("kc_rmsnorm_bf16", L.kc_rmsnorm_bf16(ptr(dh), ptr(dg), ptr(dx), 1, cols, 1e-5,
                                                      stream()))
    kc_abi.check("kc_gemv_int4_bf16", L.kc_gemv_int4_bf16(ptr(dp), ptr(ds), ptr(dz), ptr(dx),
                                                          ptr(dy), rows, cols, gs, stream()))
    gpu.cuda.synchronize()
    y2 = bf16_bits_to_f32(_bits(dy))
    h = bf16_bits_to_f32(hb).astype(np.float64)
    rinv = 1.0 / np.sqrt(np.mean(h ** 2) + 1e-5)
    exact = oracle.gemv_int4_f64(packed, scales, zeros.reshape(-1),
                                 bf16_bits_to_f32(gb).astype(np.float64) * h * rinv, rows, cols, gs)
    assert rel_l2(y, exact) < 1e-2
    assert rel_l2(y2, exact) < 1e-2


def test_rmsnorm_gemv_argument_errors(gpu):
    L = kc_abi.lib()
    rows, cols, gs = 64, 256, 128
    packed, scales, zeros = make_int4(rows, cols, gs, seed=1)
    dp, ds, dz = _dev(gpu, packed), _dev(gpu, scales), _dev(gpu, zeros)
    dh = _dev_bf16(gpu, normal_bf16((cols,), seed=2))
    dy = gpu.empty(rows, dtype=gpu.bfloat16, device="cuda")
    L.kc_get_last_error()
    st = L.kc_rmsnorm_gemv_int4_bf16(ptr(dh), None, 1e-5, ptr(dp), ptr(ds), ptr(dz), ptr(dy),
                                     rows, cols, gs, stream())
    assert st == 1 and b"null" in L.kc_last_error_string()
    st = L.kc_rmsnorm_gemv_int4_bf16(ptr(dh), ptr(dh), 1e-5, ptr(dp), ptr(ds), ptr(dz), ptr(dy),
                                     rows, cols + 1, gs, stream())
    assert st == 1
    L.kc_get_last_error()
    st = L.kc_rmsnorm_bf16(ptr(dh), ptr(dh), ptr(dy), -1, cols, 1e-5, stream())
    assert st == 1
    L.kc_get_last_error()


# ---------------------------------------------------------------------------
# RMSNorm -> FP8 per-token quantization (kc_rmsnorm_quantize_fp8_bf16)
# ---------------------------------------------------------------------------

def _norm_fp8(torch, hb, gb, eps=1e-6, offset=0):
    """kc_rmsnorm_quantize_fp8_bf16 through the C ABI; offset (in elements)
    moves h, gamma and the codes off their alignment (generic kernel)."""
    L = kc_abi.lib()
    T, D = hb.shape
    hbuf = torch.zeros(T * D + offset, dtype=torch.bfloat16, device="cuda")
    hbuf[offset:] = _dev_bf16(torch, hb.reshape(-1))
    gbuf = torch.zeros(D + offset, dtype=torch.bfloat16, device="cuda")
    gbuf[offset:] = _dev_bf16(torch, gb)
    qbuf = torch.full((T * D + offset,), 0x55, dtype=torch.int8, device="cuda")
    s = torch.full((T,), float("nan"), dtype=torch.float32, device="cuda")
    print(f"kc_rmsnorm_quantize_fp8_bf16 T={T} D={D} offset={offset}", flush=True)
    st = L.kc_rmsnorm_quantize_fp8_bf16(ptr(hbuf[offset:]), ptr(gbuf[offset:]), eps,
                                        ptr(qbuf[offset:]), ptr(s), T, D, stream())
    kc_abi.check("kc_rmsnorm_quantize_fp8_bf16", st)
    torch.cuda.synchronize()
    return qbuf[offset:].cpu().numpy().reshape(T, D), s.cpu().numpy()


def _special_rows(hb):
    """Rows the reference's arithmetic treats specially, planted in place."""
    T, D = hb.shape
    specials = [
        np.zeros(D, np.uint16),                                      # zero row
        np.full(D, 0x8000, np.uint16),                               # -0 row
        np.where(np.arange(D) == 3, 0x7FC0, hb[0]).astype(np.uint16),  # one quiet NaN
        np.where(np.arange(D) == 5, 0x7F81, hb[0]).astype(np.uint16),  # one signalling NaN
        np.where(np.arange(D) == 7, 0xFF80, hb[0]).astype(np.uint16),  # -inf
        f32_to_bf16_bits(np.full(D, 2.0 ** -70, np.float32)),        # tiny: absmax < 2^-60?
        np.full(D, 0x7F7F, np.uint16),                               # bf16 max: ss overflows
        np.where(np.arange(D) % 97 == 0, 0x0001, 0).astype(np.uint16),  # subnormals only
    ]
    for i, row in enumerate(specials[:T]):
        hb[i] = row
    return hb


@pytest.mark.parametrize("T", [1, 7, 4096, 16384])
@pytest.mark.parametrize("D", [4096, 8192])
def test_rmsnorm_quantize_fp8_bit_exact(gpu, oracle, T, D):
    """Codes and scales bit for bit against the oracle composition
    kco_rmsnorm_bf16_lanes -> kco_quantize_fp8_per_token_bf16, with special
    rows planted at the top (zero, -0, NaN, sNaN, -inf, tiny, overflowing,
    subnormal)."""
    hb = normal_bf16((T, D), seed=T + D, std=2.0)
    hb = _special_rows(hb)
    rng = np.random.default_rng(D)
    gb = f32_to_bf16_bits(rng.uniform(0.25, 2.0, D).astype(np.float32))
    q, s = _norm_fp8(gpu, hb, gb)
    eq, es = oracle.rmsnorm_quantize_fp8_bf16(hb, gb, 1e-6)
    np.testing.assert_array_equal(s, es)
    np.testing.assert_array_equal(q, eq)


@pytest.mark.parametrize("T,D,offset", [(5, 100, 0), (3, 4104, 1), (4, 20000, 0), (9, 512, 0),
                                        (6, 2048, 0), (2, 8, 0), (3, 1, 0), (0, 64, 0)])
def test_rmsnorm_quantize_fp8_shapes(gpu, oracle, T, D, offset):
    """Short rows, rows past 8192 values and unaligned buffers (the generic
    kernel) keep the same summation order, so the same bits."""
    hb = normal_bf16((T, D), seed=T * 7 + D, std=1.5)
    gb = f32_to_bf16_bits(np.random.default_rng(D).uniform(0.5, 1.5, D).astype(np.float32))
    q, s = _norm_fp8(gpu, hb, gb, 1e-5, offset)
    if T:
        eq, es = oracle.rmsnorm_quantize_fp8_bf16(hb, gb, 1e-5)
        np.testing.assert_array_equal(s, es)
        np.testing.assert_array_equal(q, eq)


def test_rmsnorm_quantize_fp8_equals_two_launches(gpu):
    """The fused launch equals kc_rmsnorm_bf16 followed by
    kc_quantize_fp8_per_token_bf16 on its output, bit for bit (cfg4 rows)."""
    L = kc_abi.lib()
    T, D = 512, 8192
    hb = normal_bf16((T, D), seed=77)
    gb = f32_to_bf16_bits(np.random.default_rng(78).uniform(0.5, 1.5, D).astype(np.float32))
    q, s = _norm_fp8(gpu, hb, gb, 1e-6)
    dh, dg = _dev_bf16(gpu, hb), _dev_bf16(gpu, gb)
    dy = gpu.empty(T, D, dtype=gpu.bfloat16, device="cuda")
    dq = gpu.empty(T, D, dtype=gpu.int8, device="cuda")
    ds = gpu.empty(T, dtype=gpu.float32, device="cuda")
    print("kc_rmsnorm_bf16 + kc_quantize_fp8_per_token_bf16", flush=True)
    kc_abi.check("kc_rmsnorm_bf16", L.kc_rmsnorm_bf16(ptr(dh), ptr(dg), ptr(dy), T, D, 1e-6,
                                                      stream()))
    kc_abi.check("kc_quantize_fp8_per_token_bf16",
                 L.kc_quantize_fp8_per_token_bf16(ptr(dy), ptr(dq), ptr(ds), T, D, stream()))
    gpu.cuda.synchronize()
    np.testing.assert_array_equal(q, dq.cpu().numpy())
    np.testing.assert_array_equal(s, ds.cpu().numpy())


def test_rmsnorm_quantize_fp8_argument_errors(gpu):
    L = kc_abi.lib()
    d = gpu.zeros(64, dtype=gpu.bfloat16, device="cuda")
    q = gpu.zeros(64, dtype=gpu.int8, device="cuda")
    s = gpu.zeros(1, dtype=gpu.float32, device="cuda")
    L.kc_get_last_error()
    assert L.kc_rmsnorm_quantize_fp8_bf16(ptr(d), None, 1e-6, ptr(q), ptr(s), 1, 64, stream()) == 1
    assert b"null" in L.kc_last_error_string()
    assert L.kc_rmsnorm_quantize_fp8_bf16(ptr(d), ptr(d), 1e-6, ptr(q), ptr(s), -1, 64,
                                          stream()) == 1
    L.kc_get_last_error()
    assert L.kc_rmsnorm_quantize_fp8_bf16(None, None, 1e-6, None, None, 0, 64, stream()) == 0
    assert L.kc_get_last_error() == 0
