"""FP8 E4M3 quantization on the GPU vs the CPU oracle: codes and scales
bit-exact, on the BASELINE configurations and on the edge cases."""
import ctypes
import os

import numpy as np
import pytest

import kc_abi
from kc_abi import ptr, stream
from kc_data import bf16_bits_to_f32, f32_to_bf16_bits, normal_bf16, outlier_activations

pytestmark = pytest.mark.gpu


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _dev_bf16(torch, bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


def _per_token(torch, x):
    rows, cols = x.shape
    dx = _dev(torch, x)
    dq = torch.full((rows, cols), 0x55, dtype=torch.int8, device="cuda")
    ds = torch.full((max(rows, 1),), float("nan"), dtype=torch.float32, device="cuda")
    print(f"launch_quantize_fp8 per_token rows={rows} cols={cols}", flush=True)
    kc_abi.lib().launch_quantize_fp8(ptr(dx), ptr(dq), ptr(ds), rows, cols, True, stream())
    kc_abi.check("launch_quantize_fp8")
    return dq.cpu().numpy(), ds.cpu().numpy()[:rows]


def _assert_codes_equal(q, exp):
    if not np.array_equal(q, exp):
        bad = np.argwhere(q != exp)
        r, c = bad[0]
        raise AssertionError(f"{len(bad)} code mismatches; first at {(r, c)}: "
                             f"gpu 0x{q[r, c] & 0xFF:02x} oracle 0x{exp[r, c] & 0xFF:02x}")


# ---------------------------------------------------------------------------
# BASELINE cfg1
# ---------------------------------------------------------------------------

def test_cfg1_activations_per_token(gpu, oracle):
    """X [4096, 4096] ~ N(0,1) with 1 % of channels x50: codes and scales
    bit-exact; round-trip dequantization bit-exact against the oracle's."""
    torch = gpu
    x, _ = outlier_activations(4096, 4096, 0.01, 50.0, seed=1001)
    q, s = _per_token(torch, x)
    eq, es = oracle.quantize_fp8_per_token(x)
    np.testing.assert_array_equal(s, es)
    _assert_codes_equal(q, eq)
    dq, ds = _dev(torch, q), _dev(torch, s)
    out = torch.empty(4096, 4096, dtype=torch.float32, device="cuda")
    kc_abi.lib().launch_dequantize_fp8(ptr(dq), ptr(ds), ptr(out), 4096, 4096, True, stream())
    kc_abi.check("launch_dequantize_fp8")
    np.testing.assert_array_equal(out.cpu().numpy(),
                                  oracle.dequantize_fp8(eq, es, 4096, 4096, True))


def test_cfg1_weights_per_channel(gpu, oracle):
    """W [4096, 4096] ~ N(0, 0.02): one scale per output channel (row)."""
    w = (np.random.default_rng(1002).standard_normal((4096, 4096)) * 0.02).astype(np.float32)
    q, s = _per_token(gpu, w)
    eq, es = oracle.quantize_fp8_per_token(w)
    np.testing.assert_array_equal(s, es)
    _assert_codes_equal(q, eq)


# ---------------------------------------------------------------------------
# Shapes (fast and generic paths) and special values
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 3), (2, 31), (5, 33), (4, 100), (8, 1000),
                                       (3, 1024), (3, 1028), (2, 4096), (2, 8192), (2, 8196),
                                       (2, 12000), (1, 65536)])
def test_per_token_shapes(gpu, oracle, rows, cols):
    x = (np.random.default_rng(rows * cols).standard_normal((rows, cols)) * 3).astype(np.float32)
    q, s = _per_token(gpu, x)
    eq, es = oracle.quantize_fp8_per_token(x)
    np.testing.assert_array_equal(s, es)
    _assert_codes_equal(q, eq)


def _per_token_bf16(torch, xb, smooth=None, mode="none"):
    """kc_quantize_fp8_per_token_bf16 / _smooth_div_bf16 / _smooth_mul_bf16 on
    bf16 bits xb [rows, cols]; returns (codes, scales) on the host."""
    rows, cols = xb.shape
    L = kc_abi.lib()
    dx = _dev_bf16(torch, xb)
    dq = torch.full((rows, cols), 0x55, dtype=torch.int8, device="cuda")
    ds = torch.full((max(rows, 1),), float("nan"), dtype=torch.float32, device="cuda")
    print(f"fp8 bf16 {mode} rows={rows} cols={cols}", flush=True)
    if mode == "none":
        st = L.kc_quantize_fp8_per_token_bf16(ptr(dx), ptr(dq), ptr(ds), rows, cols, stream())
    else:
        dsm = _dev(torch, smooth)
        fn = L.kc_quantize_fp8_smooth_div_bf16 if mode == "div" else L.kc_quantize_fp8_smooth_mul_bf16
        st = fn(ptr(dx), ptr(dsm), ptr(dq), ptr(ds), rows, cols, stream())
    kc_abi.check(f"fp8 bf16 {mode}", st)
    torch.cuda.synchronize()
    return dq.cpu().numpy(), ds.cpu().numpy()[:rows]


# bf16 rows: one wave per row with 1, 2, 4, 8 and 16 slots per lane (up to
# D = 8192, partial last slots included), one workgroup per row (8200, 16384),
# and the generic two-pass kernel (odd D, D > 16384).
BF16_SHAPES = [(3, 8), (2, 72), (3, 520), (2, 1024), (2, 2056), (2, 4096), (3, 8192),
               (2, 8200), (2, 16384), (2, 20000), (3, 7), (2, 1001)]


@pytest.mark.parametrize("rows,cols", BF16_SHAPES)
def test_per_token_bf16_shapes(gpu, oracle, rows, cols):
    x, _ = outlier_activations(rows, cols, 0.01, 50.0, seed=rows * 7919 + cols)
    xb = f32_to_bf16_bits(x)
    q, s = _per_token_bf16(gpu, xb)
    eq, es = oracle.quantize_fp8_per_token_bf16(xb)
    np.testing.assert_array_equal(s.view(np.uint32), es.view(np.uint32))
    _assert_codes_equal(q, eq)


# Smoothing routes: one wave per row (520), the persistent kernel for rows of
# 256..1024 16-byte slots (2048..8192: full and partial slot sets, and more
# rows than its grid), one workgroup per row (8200), the generic kernel.
@pytest.mark.parametrize("rows,cols", [(2, 520), (3, 2048), (2, 2056), (3, 4096), (4, 6152),
                                       (2, 8192), (8000, 2048), (2, 8200), (2, 20000)])
@pytest.mark.parametrize("mode", ["div", "mul"])
def test_smooth_bf16_shapes(gpu, oracle, rows, cols, mode):
    x, _ = outlier_activations(rows, cols, 0.005, 100.0, seed=rows * 131 + cols)
    xb = f32_to_bf16_bits(x)
    sm = np.random.default_rng(cols).uniform(0.05, 30.0, cols).astype(np.float32)
    q, s = _per_token_bf16(gpu, xb, sm, mode)
    if mode == "div":
        eq, es = oracle.quantize_fp8_smooth_div(xb, sm)
    else:
        eq, es = oracle.quantize_fp8_smooth_mul_bf16(xb, sm)
    np.testing.assert_array_equal(s.view(np.uint32), es.view(np.uint32))
    _assert_codes_equal(q, eq)


def _smooth_div_f32(torch, x, sm):
    rows, cols = x.shape
    L = kc_abi.lib()
    dx, dsm = _dev(torch, x), _dev(torch, sm)
    dq = torch.full((rows, cols), 0x55, dtype=torch.int8, device="cuda")
    ds = torch.full((max(rows, 1),), float("nan"), dtype=torch.float32, device="cuda")
    print(f"fp8 f32 div rows={rows} cols={cols}", flush=True)
    kc_abi.check("kc_quantize_fp8_smooth_div_f32",
                 L.kc_quantize_fp8_smooth_div_f32(ptr(dx), ptr(dsm), ptr(dq), ptr(ds), rows, cols,
                                                  stream()))
    torch.cuda.synchronize()
    return dq.cpu().numpy(), ds.cpu().numpy()[:rows]


@pytest.mark.parametrize("rows,cols", [(2, 520), (3, 1024), (2, 1028), (3, 2052), (2, 4096),
                                       (6000, 1024), (2, 4100)])
def test_smooth_div_f32_shapes(gpu, oracle, rows, cols):
    x, _ = outlier_activations(rows, cols, 0.005, 100.0, seed=rows * 17 + cols)
    sm = np.random.default_rng(cols + 1).uniform(0.05, 30.0, cols).astype(np.float32)
    q, s = _smooth_div_f32(gpu, x, sm)
    eq, es = oracle.quantize_fp8_smooth_div(x, sm)
    np.testing.assert_array_equal(s.view(np.uint32), es.view(np.uint32))
    _assert_codes_equal(q, eq)


def _special_rows(rng, cols):
    """Rows that leave the smoothing division's fast route, between ordinary
    rows: zeros, -0, NaN, infinities, quotients that overflow, all-tiny rows,
    tiny elements under a normal maximum, and a wide exponent spread."""
    x = rng.standard_normal((16, cols)).astype(np.float32)
    x[1] = 0.0
    x[2] = -0.0
    x[3, ::7] = np.nan
    x[4, 5] = np.inf
    x[5, 9] = -np.inf
    x[6] = np.float32(3e38) * rng.uniform(-1, 1, cols).astype(np.float32)    # x / s overflows
    x[7] = np.float32(2.0 ** -110) * rng.standard_normal(cols).astype(np.float32)
    x[8] = np.float32(2.0 ** -135) * np.sign(rng.standard_normal(cols)).astype(np.float32)
    x[9] = np.float32(2.0 ** -100) * rng.standard_normal(cols).astype(np.float32)
    x[9, 3] = 1.0
    x[10] = np.float32(2.0) ** rng.integers(-126, 127, cols).astype(np.float32)
    x[11, :] = np.nan
    x[12] = np.float32(2.0 ** -70) * rng.standard_normal(cols).astype(np.float32)
    x[13, ::3] = -0.0
    return x


def _special_factors(rng, cols, kind):
    if kind == "normal":
        return rng.uniform(0.05, 30.0, cols).astype(np.float32)
    if kind == "wide":
        return (np.float32(2.0) ** rng.integers(-119, 120, cols)).astype(np.float32)
    s = rng.uniform(0.05, 30.0, cols).astype(np.float32)
    s[[1, 5, 9, 13, 17, 21, 25]] = [0.0, 2.0 ** -125, np.inf, np.nan, -2.0, 2.0 ** 125, 1e-45]
    return s


@pytest.mark.parametrize("factors", ["normal", "wide", "outside"])
@pytest.mark.parametrize("dtype,cols", [("bf16", 2048), ("bf16", 4104), ("f32", 1024),
                                        ("f32", 2052)])
@pytest.mark.parametrize("mode", ["div", "mul"])
def test_smooth_special_values(gpu, oracle, mode, dtype, cols, factors):
    """Special rows and factors through the persistent smoothing kernel,
    including the rows and factor vectors that its Markstein check sends to
    the IEEE route."""
    if mode == "mul" and dtype == "f32":
        pytest.skip("the smoothing multiply takes bf16 weights")
    rng = np.random.default_rng(cols * 7 + len(factors))
    x = _special_rows(rng, cols)
    sm = _special_factors(rng, cols, factors)
    if dtype == "bf16":
        xb = f32_to_bf16_bits(x)
        q, s = _per_token_bf16(gpu, xb, sm, mode)
        if mode == "div":
            eq, es = oracle.quantize_fp8_smooth_div(xb, sm)
        else:
            eq, es = oracle.quantize_fp8_smooth_mul_bf16(xb, sm)
    else:
        q, s = _smooth_div_f32(gpu, x, sm)
        eq, es = oracle.quantize_fp8_smooth_div(x, sm)
    np.testing.assert_array_equal(s.view(np.uint32), es.view(np.uint32))
    _assert_codes_equal(q, eq)


@pytest.mark.parametrize("cols", [512, 8192])
def test_per_token_bf16_special_values(gpu, oracle, cols):
    """bf16 rows with zeros, -0, NaN, inf, denormals and tiny absmax values
    (the scale routes that divide exactly) through the one-wave kernel (512)
    and the persistent one (8192)."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((10, cols)).astype(np.float32)
    x[0] = 0.0
    x[1] = -0.0
    x[2, ::5] = np.nan
    x[3, 7] = np.inf
    x[4] = np.float32(2.0 ** -130) * np.sign(rng.standard_normal(cols)).astype(np.float32)  # denormal bf16
    x[5] = np.float32(2.0 ** -70) * rng.standard_normal(cols).astype(np.float32)          # absmax < 2^-60
    x[6] = np.float32(3e38) * rng.uniform(-1, 1, cols).astype(np.float32)
    x[7, :] = np.nan
    x[8] = np.float32(2.0 ** -100) * rng.standard_normal(cols).astype(np.float32)
    x[8, 3] = 1.0                                # tiny elements under a normal absmax
    x[9] = np.float32(2.0) ** rng.integers(-40, 40, cols).astype(np.float32)
    xb = f32_to_bf16_bits(x)
    q, s = _per_token_bf16(gpu, xb)
    eq, es = oracle.quantize_fp8_per_token_bf16(xb)
    np.testing.assert_array_equal(s.view(np.uint32), es.view(np.uint32))
    _assert_codes_equal(q, eq)


@pytest.mark.parametrize("cols", [256, 4096])
def test_per_token_special_values(gpu, oracle, cols):
    """One-wave kernel (256) and persistent kernel (4096 columns)."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((15, cols)).astype(np.float32)
    x[0] = 0.0                                   # all zero -> scale 1
    x[1] = -0.0                                  # -0 -> code 0x80
    x[2, ::7] = np.nan                           # NaN ignored by absmax, -> +448
    x[3, 5] = np.inf                             # inf row -> scale inf
    x[4, 9] = -np.inf
    x[5] = np.float32(1e-42)                     # denormal absmax -> denormal scale
    x[5, ::2] = np.float32(-1e-42)
    x[6] = rng.uniform(-1, 1, cols).astype(np.float32) * np.float32(3e38)   # huge, finite
    x[7] = np.float32(2.0 ** -126) * rng.standard_normal(cols).astype(np.float32)
    x[8, :] = np.nan                             # all NaN -> scale 1, codes +448
    x[9] = rng.standard_normal(cols).astype(np.float32) * np.float32(1e-30)
    x[10, 0] = np.float32(448.0)                 # exact max
    x[11] = np.float32(2.0) ** rng.integers(-20, 20, cols).astype(np.float32)
    x[12] = np.float32(1e-44) * np.sign(rng.standard_normal(cols)).astype(np.float32)  # scale 0
    x[12, 3] = 0.0
    snan = np.array([0x7F800001, 0x7FA00000, 0xFF800001, 0xFFBFFFFF], np.uint32).view(np.float32)
    x[13, :4] = snan                             # signaling NaNs: ignored, -> +448
    x[14, 10:14] = snan
    q, s = _per_token(gpu, x)
    eq, es = oracle.quantize_fp8_per_token(x)
    np.testing.assert_array_equal(s.view(np.uint32), es.view(np.uint32))
    _assert_codes_equal(q, eq)


@pytest.mark.parametrize("cols", [512, 4096])
def test_per_token_rounding_boundaries(gpu, oracle, cols):
    """Inputs whose quotient x/scale lands on E4M3 rounding midpoints and on
    their fp32 neighbours: the divide must be correctly rounded (one-wave
    kernel at 512 columns, persistent kernel at 4096)."""
    rng = np.random.default_rng(11)
    table = oracle.e4m3_decode_table()
    pos = np.sort(table[:0x7F])                       # finite non-negative values
    mids = ((pos[1:].astype(np.float64) + pos[:-1]) / 2).astype(np.float32)
    rows = []
    for _ in range(64):
        amax = np.float32(rng.uniform(0.1, 100.0))
        scale = np.float32(amax / np.float32(448.0))
        vals = (mids.astype(np.float64) * np.float64(scale)).astype(np.float32)
        vals = np.concatenate([vals, np.nextafter(vals, np.float32(np.inf)),
                               np.nextafter(vals, np.float32(0))])
        row = np.resize(vals, cols).astype(np.float32)
        row *= np.where(rng.random(cols) < 0.5, -1, 1).astype(np.float32)
        row[0] = amax
        rows.append(row)
    x = np.stack(rows)
    q, s = _per_token(gpu, x)
    eq, es = oracle.quantize_fp8_per_token(x)
    np.testing.assert_array_equal(s, es)
    _assert_codes_equal(q, eq)


def test_reference_kats_roundtrip(gpu, golden):
    """test_fp8_quant.cpp:34-71 and test_transformer_bindings.py:212-220."""
    torch = gpu
    for name in ("fp8_tok_srand42_x", "fp8_tok_rng42_x", "fp8_tok_rng11_x"):
        x = golden[name]
        q, s = _per_token(torch, x)
        out = torch.empty(*x.shape, dtype=torch.float32, device="cuda")
        dq, ds = _dev(torch, q), _dev(torch, s)      # keep alive across the launch
        kc_abi.lib().launch_dequantize_fp8(ptr(dq), ptr(ds), ptr(out),
                                           x.shape[0], x.shape[1], True, stream())
        kc_abi.check("launch_dequantize_fp8")
        xh = out.cpu().numpy()
        nz = np.abs(x) > 1e-6
        assert np.max(np.abs(xh[nz] - x[nz]) / np.abs(x[nz])) < 0.15
    q, s = _per_token(torch, np.zeros((4, 32), np.float32))
    assert np.all(q == 0) and np.all(s == 1.0)


# ---------------------------------------------------------------------------
# Per-tensor, including the exhaustive conversion sweep
# ---------------------------------------------------------------------------

def _per_tensor(torch, dx, scale_value, rows, cols, x_offset_bytes=0):
    dq = torch.full((rows * cols,), 0x55, dtype=torch.int8, device="cuda")
    ds = torch.tensor([scale_value], dtype=torch.float32, device="cuda")
    kc_abi.lib().launch_quantize_fp8(ctypes.c_void_p(dx.data_ptr() + x_offset_bytes), ptr(dq),
                                     ptr(ds), rows, cols, False, stream())
    kc_abi.check("launch_quantize_fp8")
    return dq


def test_per_tensor_reference_kat(gpu, oracle, golden):
    torch = gpu
    x = golden["fp8_tensor_srand7_x"]
    scale = float(golden["fp8_tensor_srand7_scale"][0])
    q = _per_tensor(torch, _dev(torch, x), scale, *x.shape).cpu().numpy().reshape(x.shape)
    _assert_codes_equal(q, oracle.quantize_fp8_per_tensor(x, scale))


@pytest.mark.parametrize("n,offset", [(4096 * 257, 0), (1001, 0), (1003, 4)])
def test_per_tensor_shapes_and_alignment(gpu, oracle, n, offset):
    torch = gpu
    x = (np.random.default_rng(n).standard_normal(n + 1) * 10).astype(np.float32)
    dx = _dev(torch, x)
    xs = x[offset // 4: offset // 4 + n]
    q = _per_tensor(torch, dx, 0.037, 1, n, offset).cpu().numpy()
    _assert_codes_equal(q.reshape(1, n), oracle.quantize_fp8_per_tensor(xs, 0.037).reshape(1, n))


def test_per_tensor_zero_scale_saturates(gpu):
    """Reference quirk: the ctypes bridge passes a zeroed scale buffer."""
    torch = gpu
    x = torch.tensor([[1.0, -1.0, 0.0, -0.0, 3.0]], dtype=torch.float32, device="cuda")
    q = _per_tensor(torch, x, 0.0, 1, 5).cpu().numpy().view(np.uint8)
    assert list(q) == [0x7E, 0xFE, 0x7E, 0x7E, 0x7E]


def test_e4m3_conversion_exhaustive(gpu, oracle):
    """Every one of the 2^32 fp32 bit patterns through the product's own
    clamp + v_cvt_pk_fp8_f32 path (per-tensor quantization with scale 1, for
    which x / 1 == x), against the oracle's OCP encoder."""
    torch = gpu
    chunk = 1 << 28
    for start in range(0, 1 << 32, chunk):
        bits = torch.arange(start, start + chunk, dtype=torch.int64, device="cuda")
        bits = torch.where(bits >= 2 ** 31, bits - 2 ** 32, bits)   # same 32 bits, signed
        x = bits.to(torch.int32).view(torch.float32)
        del bits
        q = _per_tensor(torch, x, 1.0, 1, chunk).cpu().numpy().view(np.uint8)
        del x
        print(f"e4m3 sweep chunk 0x{start:08x}", flush=True)
        bad, first = oracle.sweep_mismatches(start, q)
        assert bad == 0, f"{bad} mismatches from 0x{start:08x}, first 0x{first:08x}"


def test_dequant_all_codes(gpu, oracle):
    torch = gpu
    q = np.tile(np.arange(256, dtype=np.uint8), 8).view(np.int8).reshape(4, 512)
    s = np.array([1.0, 0.5, 3.7e-3, 1e30], np.float32)
    out = torch.empty(4, 512, dtype=torch.float32, device="cuda")
    L = kc_abi.lib()
    dq, ds = _dev(torch, q), _dev(torch, s)
    L.launch_dequantize_fp8(ptr(dq), ptr(ds), ptr(out), 4, 512, True, stream())
    kc_abi.check("launch_dequantize_fp8")
    got = out.cpu().numpy()
    exp = oracle.dequantize_fp8(q, s, 4, 512, True)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(exp))
    np.testing.assert_array_equal(got[~np.isnan(exp)], exp[~np.isnan(exp)])
    # per-tensor mode and ragged columns (generic tail)
    q2 = q.reshape(-1)[:3 * 7].reshape(3, 7)
    out2 = torch.empty(3, 7, dtype=torch.float32, device="cuda")
    dq2 = _dev(torch, q2)
    L.launch_dequantize_fp8(ptr(dq2), ptr(ds), ptr(out2), 3, 7, False, stream())
    kc_abi.check("launch_dequantize_fp8")
    exp2 = oracle.dequantize_fp8(q2, s, 3, 7, False)
    np.testing.assert_array_equal(out2.cpu().numpy(), exp2)


def test_reference_launchers_empty_shapes(gpu):
    L = kc_abi.lib()
    L.kc_get_last_error()
    L.launch_quantize_fp8(None, None, None, 0, 64, True, stream())
    L.launch_dequantize_fp8(None, None, None, 0, 64, True, stream())
    L.launch_smoothquant_scale(None, None, None, 0, 64, stream())
    assert L.kc_get_last_error() == 0


# ---------------------------------------------------------------------------
# SmoothQuant
# ---------------------------------------------------------------------------

def test_smoothquant_scale_kat_and_random(gpu, oracle, golden):
    torch = gpu
    L = kc_abi.lib()
    for x, s in [(golden["smooth_kat_x"], golden["smooth_kat_s"]),
                 (np.random.default_rng(1).standard_normal((33, 1000)).astype(np.float32),
                  np.random.default_rng(2).uniform(0.1, 50, 1000).astype(np.float32)),
                 (np.random.default_rng(3).standard_normal((5, 37)).astype(np.float32),
                  np.random.default_rng(4).uniform(0.1, 50, 37).astype(np.float32))]:
        out = torch.empty(*x.shape, dtype=torch.float32, device="cuda")
        dx, ds = _dev(torch, x), _dev(torch, s)
        L.launch_smoothquant_scale(ptr(dx), ptr(ds), ptr(out), x.shape[0], x.shape[1], stream())
        kc_abi.check("launch_smoothquant_scale")
        np.testing.assert_array_equal(out.cpu().numpy(), oracle.smoothquant_scale(x, s))


def _smooth_pipeline(torch, xb, wb):
    """Stats pass, factors, then the single-pass quantizers (cfg4)."""
    L = kc_abi.lib()
    T, D = xb.shape
    N = wb.shape[0]
    ax = torch.empty(D, dtype=torch.float32, device="cuda")
    aw = torch.empty(D, dtype=torch.float32, device="cuda")
    s = torch.empty(D, dtype=torch.float32, device="cuda")
    for st in (L.kc_col_absmax_bf16(ptr(xb), ptr(ax), T, D, stream()),
               L.kc_col_absmax_bf16(ptr(wb), ptr(aw), N, D, stream()),
               L.kc_smooth_factors(ptr(ax), ptr(aw), ptr(s), D, stream())):
        kc_abi.check("smoothquant stats", st)
    qx = torch.empty(T, D, dtype=torch.int8, device="cuda")
    sx = torch.empty(T, dtype=torch.float32, device="cuda")
    qw = torch.empty(N, D, dtype=torch.int8, device="cuda")
    sw = torch.empty(N, dtype=torch.float32, device="cuda")
    kc_abi.check("kc_quantize_fp8_smooth_div_bf16",
                 L.kc_quantize_fp8_smooth_div_bf16(ptr(xb), ptr(s), ptr(qx), ptr(sx), T, D, stream()))
    kc_abi.check("kc_quantize_fp8_smooth_mul_bf16",
                 L.kc_quantize_fp8_smooth_mul_bf16(ptr(wb), ptr(s), ptr(qw), ptr(sw), N, D, stream()))
    torch.cuda.synchronize()
    return ax, aw, s, qx, sx, qw, sw


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("rows,cols", [(1, 8), (130, 2048), (257, 4104), (64, 1000), (300, 20), (7, 16392)])
def test_col_absmax_shapes(gpu, oracle, dtype, rows, cols):
    """Column absmax (SmoothQuant statistics) over band and tile tails, the
    scalar path (cols not a multiple of the 16-byte slot) and special values:
    NaN and signaling NaN are ignored, inf wins, -0 counts as 0."""
    torch = gpu
    rng = np.random.default_rng(rows * 31 + cols)
    x = (rng.standard_normal((rows, cols)) * rng.uniform(0.1, 50.0, cols)).astype(np.float32)
    x[rng.integers(0, rows, 5), rng.integers(0, cols, 5)] = np.nan
    snan = np.array([0x7F800001, 0xFFA00000], np.uint32).view(np.float32)
    x[rows - 1, 0] = snan[0]
    x[0, cols - 1] = snan[1]
    if cols > 3:
        x[:, 3] = -0.0
        x[rows // 2, 2] = -np.inf
    L = kc_abi.lib()
    out = torch.full((cols,), float("nan"), dtype=torch.float32, device="cuda")
    if dtype == "bf16":
        xb = f32_to_bf16_bits(x)
        dx = _dev_bf16(torch, xb)
        st = L.kc_col_absmax_bf16(ptr(dx), ptr(out), rows, cols, stream())
        exp = oracle.col_absmax(xb)
    else:
        dx = _dev(torch, x)
        st = L.kc_col_absmax_f32(ptr(dx), ptr(out), rows, cols, stream())
        exp = oracle.col_absmax(x)
    kc_abi.check("col_absmax", st)
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("T,N,D", [(256, 384, 8192), (1, 1, 8), (130, 257, 4104), (300, 7, 20),
                                   (0, 64, 2048), (64, 0, 2048), (5, 3, 1000)])
def test_smoothquant_stats_one_call(gpu, oracle, dtype, T, N, D):
    """kc_smoothquant_stats_* (both maxima and the factors from one call)
    equals kc_col_absmax_* on X and on W followed by kc_smooth_factors, bit
    for bit, and the oracle: band and tile tails, the scalar path (cols not a
    multiple of the 16-byte slot), empty X or W, NaN, signaling NaN and inf."""
    torch = gpu
    L = kc_abi.lib()
    rng = np.random.default_rng(T * 7 + N * 13 + D)
    x = (rng.standard_normal((T, D)) * rng.uniform(0.1, 50.0, D)).astype(np.float32)
    w = (rng.standard_normal((N, D)) * 0.02).astype(np.float32)
    if T > 2 and D > 4:
        x[1, 2] = np.nan
        x[T - 1, 0] = np.array([0x7F800001], np.uint32).view(np.float32)[0]
        x[0, 3] = -np.inf
    if N > 1 and D > 5:
        w[N - 1, 5] = np.array([0xFFA00000], np.uint32).view(np.float32)[0]
    if dtype == "bf16":
        xh, wh = f32_to_bf16_bits(x), f32_to_bf16_bits(w)
        dx, dw = _dev_bf16(torch, xh), _dev_bf16(torch, wh)
        fused, absmax = L.kc_smoothquant_stats_bf16, L.kc_col_absmax_bf16
    else:
        xh, wh = x, w
        dx, dw = _dev(torch, x), _dev(torch, w)
        fused, absmax = L.kc_smoothquant_stats_f32, L.kc_col_absmax_f32
    out = [torch.full((D,), float("nan"), dtype=torch.float32, device="cuda") for _ in range(6)]
    kc_abi.check("kc_smoothquant_stats", fused(ptr(dx), T, ptr(dw), N, D, ptr(out[0]), ptr(out[1]),
                                               ptr(out[2]), stream()))
    for st in (absmax(ptr(dx), ptr(out[3]), T, D, stream()), absmax(ptr(dw), ptr(out[4]), N, D, stream()),
               L.kc_smooth_factors(ptr(out[3]), ptr(out[4]), ptr(out[5]), D, stream())):
        kc_abi.check("three-call statistics", st)
    got = [o.cpu().numpy() for o in out]
    for a, b in zip(got[:3], got[3:]):
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    eax = oracle.col_absmax(xh) if T else np.zeros(D, np.float32)
    eaw = oracle.col_absmax(wh) if N else np.zeros(D, np.float32)
    np.testing.assert_array_equal(got[0].view(np.uint32), eax.view(np.uint32))
    np.testing.assert_array_equal(got[1].view(np.uint32), eaw.view(np.uint32))
    np.testing.assert_array_equal(got[2], oracle.smooth_factors(eax, eaw))


def test_smoothquant_stats_cfg4_bridge(gpu):
    """The bridge op on cfg4's full shapes (X [16384, 8192], W [28672, 8192]
    bf16) against the three-call statistics on the same device tensors."""
    torch = gpu
    import kernel_craft_torch_ops as ops
    g = torch.Generator(device="cuda")
    g.manual_seed(4004)
    X = torch.randn(16384, 8192, device="cuda", generator=g).to(torch.bfloat16)
    X[:, ::200] *= 100
    W = (torch.randn(28672, 8192, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    ax, aw, s = ops.smoothquant_stats(X, W)
    ex, ew = ops.col_absmax(X), ops.col_absmax(W)
    es = ops.smooth_factors(ex, ew)
    assert torch.equal(ax, ex) and torch.equal(aw, ew) and torch.equal(s, es)
    assert torch.equal(ax, X.float().abs().amax(0)) and torch.equal(aw, W.float().abs().amax(0))


def test_smoothquant_fused_small(gpu, oracle):
    """cfg4 distributions at a size the oracle runs in seconds; every output
    bit-exact (absmax, factors, codes, scales)."""
    torch = gpu
    T, D, N = 256, 8192, 384
    x, _ = outlier_activations(T, D, 0.005, 100.0, seed=4001)
    xb = f32_to_bf16_bits(x)
    wb = normal_bf16((N, D), seed=4002, std=0.02)
    ax, aw, s, qx, sx, qw, sw = _smooth_pipeline(torch, _dev_bf16(torch, xb), _dev_bf16(torch, wb))
    eax, eaw = oracle.col_absmax(xb), oracle.col_absmax(wb)
    np.testing.assert_array_equal(ax.cpu().numpy(), eax)
    np.testing.assert_array_equal(aw.cpu().numpy(), eaw)
    es = oracle.smooth_factors(eax, eaw)
    np.testing.assert_array_equal(s.cpu().numpy(), es)
    eqx, esx = oracle.quantize_fp8_smooth_div(xb, es)
    np.testing.assert_array_equal(sx.cpu().numpy(), esx)
    _assert_codes_equal(qx.cpu().numpy(), eqx)
    eqw, esw = oracle.quantize_fp8_smooth_mul_bf16(wb, es)
    np.testing.assert_array_equal(sw.cpu().numpy(), esw)
    _assert_codes_equal(qw.cpu().numpy(), eqw)


def test_smoothquant_fused_equals_reference_two_launch(gpu, oracle):
    """The fused fp32 kernel against the reference's own two-launch pipeline
    (launch_smoothquant_scale then launch_quantize_fp8), both on the GPU."""
    torch = gpu
    L = kc_abi.lib()
    x, _ = outlier_activations(512, 4096, 0.005, 100.0, seed=4003)
    s = np.random.default_rng(4004).uniform(0.05, 30.0, 4096).astype(np.float32)
    dx, ds = _dev(torch, x), _dev(torch, s)
    tmp = torch.empty_like(dx)
    L.launch_smoothquant_scale(ptr(dx), ptr(ds), ptr(tmp), 512, 4096, stream())
    q2 = torch.empty(512, 4096, dtype=torch.int8, device="cuda")
    s2 = torch.empty(512, dtype=torch.float32, device="cuda")
    L.launch_quantize_fp8(ptr(tmp), ptr(q2), ptr(s2), 512, 4096, True, stream())
    kc_abi.check("two-launch")
    q1 = torch.empty_like(q2)
    s1 = torch.empty_like(s2)
    kc_abi.check("fused", L.kc_quantize_fp8_smooth_div_f32(ptr(dx), ptr(ds), ptr(q1), ptr(s1),
                                                           512, 4096, stream()))
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(s1, s2)
    eq, es = oracle.quantize_fp8_smooth_div(x, s)
    _assert_codes_equal(q1.cpu().numpy(), eq)


def test_smoothquant_cfg4_full_size(gpu, oracle):
    """Full cfg4: X bf16 [16384, 8192] (0.5 % outlier channels x100), W bf16
    [28672, 8192] ~ N(0, 0.02).  The column absmax equals torch's, the factors
    equal the oracle's on those absmax vectors, every code and scale of all
    16384 X rows and 28672 W rows equals the oracle's (its row loops split over
    the host's cores), and every row's codes decode back within the E4M3 bound."""
    torch = gpu
    T, D, N = 16384, 8192, 28672
    g = torch.Generator(device="cuda")
    g.manual_seed(4005)
    x = torch.randn(T, D, device="cuda", generator=g)
    ch = torch.randperm(D, device="cuda", generator=g)[: int(0.005 * D)]
    x[:, ch] *= 100.0
    xb = x.to(torch.bfloat16)
    del x
    wb = (torch.randn(N, D, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    ax, aw, s, qx, sx, qw, sw = _smooth_pipeline(torch, xb, wb)
    assert torch.equal(ax, xb.float().abs().amax(dim=0))
    assert torch.equal(aw, wb.float().abs().amax(dim=0))
    np.testing.assert_array_equal(s.cpu().numpy(),
                                  oracle.smooth_factors(ax.cpu().numpy(), aw.cpu().numpy()))
    threads = min(16, len(os.sched_getaffinity(0)))
    sh = s.cpu().numpy()
    xbh = xb.view(torch.int16).cpu().numpy().view(np.uint16)
    print(f"cfg4: oracle X/s over {T} rows on {threads} threads", flush=True)
    eq, es = oracle.quantize_fp8_smooth_div(xbh, sh, threads=threads)
    del xbh
    _assert_codes_equal(qx.cpu().numpy(), eq)
    np.testing.assert_array_equal(sx.cpu().numpy().view(np.uint32), es.view(np.uint32))
    del eq, es
    wbh = wb.view(torch.int16).cpu().numpy().view(np.uint16)
    print(f"cfg4: oracle W*s over {N} rows on {threads} threads", flush=True)
    eq, es = oracle.quantize_fp8_smooth_mul_bf16(wbh, sh, threads=threads)
    del wbh
    _assert_codes_equal(qw.cpu().numpy(), eq)
    np.testing.assert_array_equal(sw.cpu().numpy().view(np.uint32), es.view(np.uint32))
    del eq, es
    # round trip over every row of X: |dequant - x/s| <= 2^-4 relative + half a
    # subnormal step of the row scale
    xs = xb.float() / s
    deq = qx.view(torch.float8_e4m3fn).float() * sx[:, None]
    err = (deq - xs).abs()
    bound = (xs.abs() * (2.0 ** -4) + sx[:, None] * (2.0 ** -10)) * 1.0001
    assert bool((err <= bound).all())
