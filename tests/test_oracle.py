"""Pins the CPU oracle (oracle/kc_oracle.c) before it is trusted as the checker.

Each oracle function is checked against the reference's own known-answer
tests (tests/golden/reference_kats.npz, made by
tests/golden/make_reference_kats.py from the reference tests' inputs and
expected-value expressions), against an independent library (torch's
float8_e4m3fn for the OCP encoding), or against what the mathematics fixes
(closed forms, invariants, brute force), so that a dropped term, a wrong
sign or index, or a transposed operand fails at least one test.
"""
import math

import numpy as np
import pytest
import torch

from kc_data import (bf16_bits_to_f32, f32_to_bf16_bits, make_int4, normal_bf16,
                     outlier_activations, rel_l2)


def _kat(golden, name):
    rows, cols, gs = (int(v) for v in golden[f"{name}_shape"])
    return (golden[f"{name}_packed"], golden[f"{name}_scales"], golden[f"{name}_zeros"],
            rows, cols, gs)


def _flat_zeros(z):
    return np.ascontiguousarray(z).reshape(-1)


# ---------------------------------------------------------------------------
# INT4 against the reference's own tests
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["deq_basic", "deq_multigroup", "deq_rng42"])
def test_dequant_reference_kats(oracle, golden, name):
    """test_quant_int4.cpp:35-88, :148-199; test_transformer_bindings.py:185-196.
    The expected values are single fp32 products, so equality is exact."""
    packed, scales, zeros, rows, cols, gs = _kat(golden, name)
    out = oracle.dequantize_int4(packed, scales, _flat_zeros(zeros), rows, cols, gs)
    np.testing.assert_array_equal(out, golden[f"{name}_expected"])


def test_gemv_reference_kat_srand42(oracle, golden):
    """test_quant_int4.cpp:90-146 (tolerance 1e-4 absolute there)."""
    packed, scales, zeros, rows, cols, gs = _kat(golden, "gemv_srand42")
    x = golden["gemv_srand42_x"]
    exp = golden["gemv_srand42_expected"]
    y64 = oracle.gemv_int4_f64(packed, scales, _flat_zeros(zeros), x, rows, cols, gs)
    yref = oracle.gemv_int4_refkernel_f32(packed, scales, _flat_zeros(zeros), x, rows, cols, gs)
    assert np.max(np.abs(y64 - exp)) < 1e-4
    assert np.max(np.abs(yref - exp)) < 1e-4
    assert rel_l2(y64, exp) < 1e-6


@pytest.mark.parametrize("name", ["triton_small", "triton_medium", "triton_gs64"])
def test_gemv_reference_kats_triton(oracle, golden, name):
    """test_triton_kernels.py:76-119,244-256 (rtol 1e-2, atol 5e-3 there)."""
    packed, scales, zeros, rows, cols, gs = _kat(golden, name)
    x = golden[f"{name}_x"]
    exp = golden[f"{name}_expected"]
    y64 = oracle.gemv_int4_f64(packed, scales, _flat_zeros(zeros), x, rows, cols, gs)
    assert np.allclose(y64, exp, rtol=1e-2, atol=5e-3)
    assert rel_l2(y64, exp) < 1e-5


# ---------------------------------------------------------------------------
# INT4 invariants and independent restatements
# ---------------------------------------------------------------------------

def _numpy_dequant(packed, scales, zeros_flat, rows, cols, gs):
    """Vectorized restatement written independently of the C oracle."""
    p = packed.astype(np.int32)
    q = np.empty((rows, cols), np.int32)
    q[:, 0::2] = p & 0xF
    q[:, 1::2] = p >> 4
    q = np.where(q >= 8, q - 16, q)
    G = cols // gs
    g = np.arange(cols) // gs
    zidx = np.arange(rows)[:, None] * (G // 2) + (g // 2)[None, :]
    zb = zeros_flat.astype(np.int32)[zidx]
    z = np.where((g % 2 == 0)[None, :], zb & 0xF, zb >> 4)
    s = scales.reshape(rows, G)[:, g]
    return (q - z).astype(np.float32) * s


@pytest.mark.parametrize("rows,cols,gs", [(7, 256, 128), (5, 384, 128), (3, 96, 32),
                                          (4, 64, 64), (2, 10, 2), (3, 12, 6)])
def test_dequant_matches_numpy_restatement(oracle, rows, cols, gs):
    packed, scales, zeros = make_int4(rows, cols, gs, seed=rows * 100 + cols)
    zf = _flat_zeros(zeros)
    out = oracle.dequantize_int4(packed, scales, zf, rows, cols, gs)
    np.testing.assert_array_equal(out, _numpy_dequant(packed, scales, zf, rows, cols, gs))


def test_sign_extension_not_offset(oracle):
    """0x88 with zero point 8: sext4(8) = -8, so w = (-8 - 8) * s = -16 s;
    unsigned (GPTQ-style) nibbles would give 0.  quant_int4.cu:34-48,95-96."""
    rows, cols, gs = 2, 256, 128
    packed = np.full((rows, cols // 2), 0x88, np.uint8)
    scales = np.full((rows, 2), 0.25, np.float32)
    zeros = np.full((rows, 1), 0x88, np.uint8)
    out = oracle.dequantize_int4(packed, scales, zeros.reshape(-1), rows, cols, gs)
    assert np.all(out == -4.0)


def test_zero_point_cancels_nibble(oracle):
    """Nibble 3 with zero point 3 dequantizes to exactly 0 -> y = 0."""
    rows, cols, gs = 3, 512, 128
    packed = np.full((rows, cols // 2), 0x33, np.uint8)
    scales = np.random.default_rng(0).uniform(0.005, 0.02, (rows, 4)).astype(np.float32)
    zeros = np.full((rows, 2), 0x33, np.uint8)
    x = np.random.default_rng(1).standard_normal(cols).astype(np.float32)
    y = oracle.gemv_int4_f64(packed, scales, zeros.reshape(-1), x, rows, cols, gs)
    assert np.all(y == 0.0)


def test_zero_point_group_parity(oracle):
    """Even groups use the low nibble of the zero byte, odd groups the high."""
    rows, cols, gs = 1, 256, 64   # G = 4: zero bytes [z0|z1<<4, z2|z3<<4]
    packed = np.zeros((rows, cols // 2), np.uint8)     # all weights sext4(0) = 0
    scales = np.ones((rows, 4), np.float32)
    zeros = np.array([0x21, 0x43], np.uint8)            # z = 1, 2, 3, 4
    out = oracle.dequantize_int4(packed, scales, zeros, rows, cols, gs)
    for g, z in enumerate([1, 2, 3, 4]):
        assert np.all(out[0, g * gs:(g + 1) * gs] == -z)


def test_zero_row_stride_is_floor(oracle):
    """G odd: row r's zero bytes start at r * floor(G/2) (quant_int4.cu:93)."""
    rows, cols, gs = 3, 96, 32   # G = 3, floor(G/2) = 1
    packed = np.zeros((rows, cols // 2), np.uint8)
    scales = np.ones((rows, 3), np.float32)
    zeros = np.array([0x21, 0x43, 0x65, 0x07], np.uint8)
    out = oracle.dequantize_int4(packed, scales, zeros, rows, cols, gs)
    # row r, group g reads byte r + g // 2
    for r in range(rows):
        for g in range(3):
            zb = int(zeros[r + g // 2])
            z = zb & 0xF if g % 2 == 0 else zb >> 4
            assert np.all(out[r, g * gs:(g + 1) * gs] == -z)


def test_gemv_brute_force_tiny(oracle):
    rows, cols, gs = 3, 8, 4
    packed, scales, zeros = make_int4(rows, cols, gs, seed=5)
    x = np.random.default_rng(6).standard_normal(cols).astype(np.float32)
    y = oracle.gemv_int4_f64(packed, scales, zeros.reshape(-1), x, rows, cols, gs)
    G = cols // gs
    for r in range(rows):
        acc = 0.0
        for k in range(cols):
            byte = int(packed[r, k // 2])
            nib = (byte >> 4) if k % 2 else (byte & 0xF)
            q = nib - 16 if nib >= 8 else nib
            g = k // gs
            zb = int(zeros.reshape(-1)[r * (G // 2) + g // 2])
            z = (zb >> 4) if g % 2 else (zb & 0xF)
            w = float(np.float32(q - z) * np.float32(scales[r, g]))
            acc += w * float(x[k])
        assert math.isclose(y[r], acc, rel_tol=1e-12, abs_tol=1e-12)


def test_gemv_linearity_and_matmul(oracle):
    rows, cols, gs = 16, 1024, 128
    packed, scales, zeros = make_int4(rows, cols, gs, seed=11)
    zf = zeros.reshape(-1)
    rng = np.random.default_rng(12)
    x1 = rng.standard_normal(cols).astype(np.float32)
    x2 = rng.standard_normal(cols).astype(np.float32)
    y1 = oracle.gemv_int4_f64(packed, scales, zf, x1, rows, cols, gs)
    y2 = oracle.gemv_int4_f64(packed, scales, zf, x2, rows, cols, gs)
    y12 = oracle.gemv_int4_f64(packed, scales, zf, (x1 + x2).astype(np.float32), rows, cols, gs)
    # x1 + x2 is rounded to fp32 once per element, so compare at that level
    assert rel_l2(y12, y1 + y2) < 1e-6
    W = oracle.dequantize_int4(packed, scales, zf, rows, cols, gs).astype(np.float64)
    np.testing.assert_allclose(y1, W @ x1.astype(np.float64), rtol=1e-12, atol=1e-12)
    assert np.all(oracle.gemv_int4_f64(packed, scales, zf, np.zeros(cols, np.float32),
                                       rows, cols, gs) == 0.0)


def test_refkernel_order_within_tolerance(oracle):
    """The reference kernel's fp32 order stays within 1e-5 of the fp64 truth
    at the cfg0 distribution (here 256 x 4096)."""
    rows, cols, gs = 256, 4096, 128
    packed, scales, zeros = make_int4(rows, cols, gs, seed=0)
    x = np.random.default_rng(1).standard_normal(cols).astype(np.float32)
    zf = zeros.reshape(-1)
    y64 = oracle.gemv_int4_f64(packed, scales, zf, x, rows, cols, gs)
    y32 = oracle.gemv_int4_refkernel_f32(packed, scales, zf, x, rows, cols, gs)
    assert rel_l2(y32, y64) < 1e-5


def test_gemm_is_gemv_per_row(oracle):
    rows, cols, gs, m = 8, 512, 128, 3
    packed, scales, zeros = make_int4(rows, cols, gs, seed=21)
    zf = zeros.reshape(-1)
    xb = f32_to_bf16_bits(np.random.default_rng(22).standard_normal((m, cols)).astype(np.float32))
    Y = oracle.gemm_int4_bf16_f64(packed, scales, zf, xb, m, rows, cols, gs)
    for i in range(m):
        y = oracle.gemv_int4_f64(packed, scales, zf, bf16_bits_to_f32(xb[i]), rows, cols, gs)
        np.testing.assert_array_equal(Y[i], y)
    y32 = oracle.gemv_int4_bf16_f32(packed, scales, zf, xb[0], rows, cols, gs)
    assert rel_l2(y32, Y[0]) < 1e-5


# ---------------------------------------------------------------------------
# E4M3 encoding: OCP spec, cross-checked against torch.float8_e4m3fn
# ---------------------------------------------------------------------------

def _torch_e4m3(bits_u32: np.ndarray) -> np.ndarray:
    f = torch.from_numpy(bits_u32.view(np.float32).copy())
    return f.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_special_cases(oracle):
    enc = oracle.e4m3_encode
    assert enc(0.0) == 0x00 and enc(-0.0) == 0x80
    assert enc(448.0) == 0x7E and enc(-448.0) == 0xFE
    assert enc(2.0 ** -9) == 0x01 and enc(-(2.0 ** -9)) == 0x81
    assert enc(2.0 ** -10) == 0x00                      # tie -> even (0)
    assert enc(3 * 2.0 ** -10) == 0x02                  # 1.5 units -> 2 (even)
    assert enc(2.0 ** -6) == 0x08                       # min normal
    assert enc(1.0) == 0x38 and enc(1.0625) == 0x38     # 1 + 1/16: tie -> even
    assert enc(1.1875) == 0x3A                          # 1 + 3/16: tie -> even (1.25)
    assert enc(464.0) == 0x7E and enc(1e30) == 0x7E     # saturate to finite
    assert enc(float("inf")) == 0x7E and enc(float("-inf")) == 0xFE
    assert enc(float("nan")) & 0x7F == 0x7F


def test_e4m3_decode_table_matches_torch(oracle):
    table = oracle.e4m3_decode_table()
    ref = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn)
    ref = ref.to(torch.float32).numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(table), nan)
    assert set(np.flatnonzero(nan)) == {0x7F, 0xFF}
    np.testing.assert_array_equal(table[~nan], ref[~nan])


def test_gemm_fp8_oracle_brute_force_and_torch(oracle):
    """The W8A8 GEMM oracle: against a scalar triple loop on a tiny case, and
    against torch's float8_e4m3fn decode + fp64 matmul with the scales
    applied on the other side."""
    rng = np.random.default_rng(5)
    M, N, K = 3, 4, 16
    qx = rng.integers(0, 256, (M, K), dtype=np.uint8)
    qw = rng.integers(0, 256, (N, K), dtype=np.uint8)
    qx[(qx & 0x7F) == 0x7F] = 1
    qw[(qw & 0x7F) == 0x7F] = 2
    sx = rng.uniform(0.1, 2, M).astype(np.float32)
    sw = rng.uniform(0.1, 2, N).astype(np.float32)
    y = oracle.gemm_fp8_w8a8_f64(qx.view(np.int8), sx, qw.view(np.int8), sw)
    table = oracle.e4m3_decode_table()
    for m in range(M):
        for n in range(N):
            acc = sum(float(table[qx[m, k]]) * float(table[qw[n, k]]) for k in range(K))
            assert y[m, n] == pytest.approx(float(sx[m]) * float(sw[n]) * acc, rel=1e-13, abs=1e-300)
    qx = rng.integers(0, 256, (40, 96), dtype=np.uint8)
    qw = rng.integers(0, 256, (24, 96), dtype=np.uint8)
    qx[(qx & 0x7F) == 0x7F] = 0
    qw[(qw & 0x7F) == 0x7F] = 0
    sx = rng.uniform(0.1, 2, 40).astype(np.float32)
    sw = rng.uniform(0.1, 2, 24).astype(np.float32)
    a = torch.from_numpy(qx).view(torch.float8_e4m3fn).double() * torch.from_numpy(sx).double()[:, None]
    b = torch.from_numpy(qw).view(torch.float8_e4m3fn).double() * torch.from_numpy(sw).double()[:, None]
    np.testing.assert_allclose(oracle.gemm_fp8_w8a8_f64(qx.view(np.int8), sx, qw.view(np.int8), sw),
                               (a @ b.T).numpy(), rtol=1e-12, atol=1e-12)


def _boundary_dense_patterns():
    """Every fp32 magnitude <= 448 whose low 14 mantissa bits are one of a few
    values on either side of the E4M3 rounding points (which sit at bit 19 for
    normals and at bits 20..23 for subnormal results), both signs."""
    hi = np.arange(0, (0x43E00000 >> 14) + 1, dtype=np.uint32) << 14
    lows = np.array([0, 1, 0x1FFF, 0x2000, 0x2001, 0x3FFF], np.uint32)
    mags = (hi[:, None] | lows[None, :]).reshape(-1)
    mags = mags[mags <= 0x43E00000]
    return np.concatenate([mags, mags | np.uint32(0x80000000)])


def test_e4m3_encoder_matches_torch_boundary_dense(oracle):
    bits = _boundary_dense_patterns()
    codes = _torch_e4m3(bits)
    # every 97th block of 2^14 consecutive patterns, both signs
    mism = 0
    for h in range(0, (0x43E00000 >> 14) + 1, 97):
        start = h << 14
        rng_bits = np.arange(start, start + (1 << 14), dtype=np.uint32)
        for sign in (0, 0x80000000):
            b = rng_bits | np.uint32(sign)
            bad, _ = oracle.sweep_mismatches(int(b[0]), _torch_e4m3(b))
            mism += bad
    assert mism == 0
    # and the boundary-dense set, one pattern at a time through the encoder
    enc = np.frombuffer(bytes(oracle.lib().kco_e4m3_encode(float(f))
                              for f in bits.view(np.float32)), np.uint8)
    assert np.array_equal(enc, codes)


@pytest.mark.slow
def test_e4m3_encoder_matches_torch_exhaustive(oracle):
    """All 2.27e9 fp32 patterns with |x| <= 448 (about a minute)."""
    top = 0x43E00000
    chunk = 1 << 26
    for sign in (0, 0x80000000):
        for start in range(0, top + 1, chunk):
            n = min(chunk, top + 1 - start)
            b = np.arange(start, start + n, dtype=np.uint32) | np.uint32(sign)
            bad, first = oracle.sweep_mismatches(int(b[0]), _torch_e4m3(b))
            assert bad == 0, hex(first)


# ---------------------------------------------------------------------------
# FP8 quantization
# ---------------------------------------------------------------------------

def _torch_per_token(x: np.ndarray):
    """Independent per-token restatement with torch ops (NaN-free input)."""
    t = torch.from_numpy(x)
    amax = t.abs().amax(dim=1)
    scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = torch.clamp(t / scale[:, None], -448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(torch.int8).numpy(), scale.numpy()


def test_per_token_matches_torch_restatement(oracle):
    x, _ = outlier_activations(64, 4096, 0.01, 50.0, seed=1)
    q, s = oracle.quantize_fp8_per_token(x)
    tq, ts = _torch_per_token(x)
    np.testing.assert_array_equal(s, ts)
    np.testing.assert_array_equal(q, tq)


def test_per_token_weight_distribution(oracle):
    w = (np.random.default_rng(3).standard_normal((128, 4096)) * 0.02).astype(np.float32)
    q, s = oracle.quantize_fp8_per_token(w)
    tq, ts = _torch_per_token(w)
    np.testing.assert_array_equal(s, ts)
    np.testing.assert_array_equal(q, tq)


@pytest.mark.parametrize("name", ["fp8_tok_srand42_x", "fp8_tok_rng42_x", "fp8_tok_rng11_x"])
def test_per_token_reference_roundtrip_bound(oracle, golden, name):
    """test_fp8_quant.cpp:34-71, test_transformer_bindings.py:212-220,
    test_vllm_backend.py:214-223: round-trip relative error < 15 %."""
    x = golden[name]
    q, s = oracle.quantize_fp8_per_token(x)
    xh = oracle.dequantize_fp8(q, s, *x.shape, per_token=True)
    nz = np.abs(x) > 1e-6
    assert np.max(np.abs(xh[nz] - x[nz]) / np.abs(x[nz])) < 0.15


def test_per_tensor_reference_roundtrip_bound(oracle, golden):
    """test_fp8_quant.cpp:137-174."""
    x = golden["fp8_tensor_srand7_x"]
    scale = golden["fp8_tensor_srand7_scale"]
    q = oracle.quantize_fp8_per_tensor(x, scale[0])
    xh = oracle.dequantize_fp8(q, scale, *x.shape, per_token=False)
    nz = np.abs(x) > 1e-6
    assert np.max(np.abs(xh[nz] - x[nz]) / np.abs(x[nz])) < 0.15


def test_zero_rows_and_specials(oracle):
    """All-zero row -> scale 1 and codes 0 (test_fp8_quant.cpp:73-97);
    NaN ignored by the absmax and clamped to +448; -0 keeps its sign."""
    x = np.zeros((4, 32), np.float32)
    x[1, 3] = np.nan
    x[2, :] = -0.0
    x[3, :] = 1.0
    x[3, 5] = np.nan
    x[3, 6] = -2.0
    q, s = oracle.quantize_fp8_per_token(x)
    assert s[0] == 1.0 and s[1] == 1.0 and s[2] == 1.0
    assert s[3] == np.float32(2.0) / np.float32(448.0)
    assert np.all(q[0] == 0) and np.all(q[2].view(np.uint8) == 0x80)
    assert q[1, 3].view(np.uint8) == 0x7E and q[3, 5].view(np.uint8) == 0x7E
    assert q[3, 6].view(np.uint8) == 0xFE
    assert q[3, 0].view(np.uint8) == oracle.e4m3_encode(np.float32(1.0) / s[3])


def test_nan_follows_cuda_fmaxf_semantics(oracle):
    """CUDA's fmaxf/fminf (fp8_quant.cu:105,127) ignore a NaN operand, quiet or
    signaling: every one of the 2^24 - 2 NaN bit patterns clamps to +448, and
    a signaling NaN never interrupts a row's absmax (glibc's maxNum would turn
    it into a quiet NaN and restart the maximum after it)."""
    for start in (0x7F800001, 0xFF800001):
        n = 0x7FFFFF
        bad, first = oracle.sweep_mismatches(start, np.full(n, 0x7E, np.uint8))
        assert bad == 0, hex(first)
    snan = np.array([0x7F800001], np.uint32).view(np.float32)[0]
    x = np.array([[3.0, 1.0, snan, 2.0], [snan, snan, snan, snan]], np.float32)
    q, s = oracle.quantize_fp8_per_token(x)
    assert s[0] == np.float32(3.0) / np.float32(448.0) and s[1] == 1.0
    assert q[0, 2].view(np.uint8) == 0x7E and np.all(q[1].view(np.uint8) == 0x7E)


def test_per_tensor_zero_scale_saturates(oracle):
    """Via ctypes the reference passes scale 0 (kernel_craft_torch_ops.py:347):
    x/0 is +-inf (or NaN for 0/0), clamped to +-448 (or +448)."""
    x = np.array([[1.0, -1.0, 0.0, -0.0]], np.float32)
    q = oracle.quantize_fp8_per_tensor(x, 0.0).view(np.uint8)
    assert list(q[0]) == [0x7E, 0xFE, 0x7E, 0x7E]


def test_dequant_is_decode_times_scale(oracle):
    q = np.arange(256, dtype=np.uint8).view(np.int8).reshape(2, 128)
    s = np.array([0.5, 3.0], np.float32)
    out = oracle.dequantize_fp8(q, s, 2, 128, per_token=True)
    table = oracle.e4m3_decode_table()
    exp = np.stack([table[:128] * s[0], table[128:] * s[1]])
    np.testing.assert_array_equal(np.isnan(out), np.isnan(exp))
    ok = ~np.isnan(exp)
    np.testing.assert_array_equal(out[ok], exp[ok])


def test_smoothquant_reference_kat(oracle, golden):
    """test_fp8_quant.cpp:99-135: 100/100 = 1 and 1/1 = 1."""
    out = oracle.smoothquant_scale(golden["smooth_kat_x"], golden["smooth_kat_s"])
    np.testing.assert_array_equal(out, golden["smooth_kat_expected"])


def test_smoothquant_matches_numpy(oracle):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((16, 100)).astype(np.float32)
    s = rng.uniform(0.1, 10, 100).astype(np.float32)
    np.testing.assert_array_equal(oracle.smoothquant_scale(x, s), x / s[None, :])


# ---------------------------------------------------------------------------
# Extensions: composition identities with the pinned functions
# ---------------------------------------------------------------------------

def test_fused_smooth_div_equals_two_step(oracle):
    x, _ = outlier_activations(32, 1024, 0.005, 100.0, seed=4)
    s = np.random.default_rng(5).uniform(0.5, 20.0, 1024).astype(np.float32)
    q1, s1 = oracle.quantize_fp8_smooth_div(x, s)
    q2, s2 = oracle.quantize_fp8_per_token(oracle.smoothquant_scale(x, s))
    np.testing.assert_array_equal(q1, q2)
    np.testing.assert_array_equal(s1, s2)
    xb = f32_to_bf16_bits(x)
    q3, s3 = oracle.quantize_fp8_smooth_div(xb, s)
    q4, s4 = oracle.quantize_fp8_per_token(oracle.smoothquant_scale(bf16_bits_to_f32(xb), s))
    np.testing.assert_array_equal(q3, q4)
    np.testing.assert_array_equal(s3, s4)


def test_fused_smooth_mul_equals_two_step(oracle):
    wb = f32_to_bf16_bits((np.random.default_rng(6).standard_normal((64, 512)) * 0.02)
                          .astype(np.float32))
    s = np.random.default_rng(7).uniform(0.5, 20.0, 512).astype(np.float32)
    q1, s1 = oracle.quantize_fp8_smooth_mul_bf16(wb, s)
    q2, s2 = oracle.quantize_fp8_per_token(bf16_bits_to_f32(wb) * s[None, :])
    np.testing.assert_array_equal(q1, q2)
    np.testing.assert_array_equal(s1, s2)


def test_bf16_per_token_equals_widened_fp32(oracle):
    xb = f32_to_bf16_bits(np.random.default_rng(8).standard_normal((8, 300)).astype(np.float32))
    q1, s1 = oracle.quantize_fp8_per_token_bf16(xb)
    q2, s2 = oracle.quantize_fp8_per_token(bf16_bits_to_f32(xb))
    np.testing.assert_array_equal(q1, q2)
    np.testing.assert_array_equal(s1, s2)


def test_col_absmax_and_smooth_factors(oracle):
    x, ch = outlier_activations(64, 256, 0.02, 100.0, seed=10)
    x[3, 7] = np.nan
    amax = oracle.col_absmax(x)
    np.testing.assert_array_equal(amax, np.nanmax(np.abs(x), axis=0))
    xb = f32_to_bf16_bits(x)
    np.testing.assert_array_equal(oracle.col_absmax(xb),
                                  np.nanmax(np.abs(bf16_bits_to_f32(xb)), axis=0))
    aw = np.abs(np.random.default_rng(11).standard_normal(256).astype(np.float32)) * 0.05
    aw[0] = 0.0
    s = oracle.smooth_factors(amax, aw)
    exp = np.maximum(np.sqrt(amax) / np.sqrt(np.maximum(aw, np.float32(1e-5))), np.float32(1e-5))
    np.testing.assert_array_equal(s, exp.astype(np.float32))
    assert np.all(s[ch] > np.median(s))          # outlier channels get the large factors


def test_smooth_factors_balance_channel_maxima(oracle):
    """alpha = 0.5 migration: after X/s and W*s every channel's maximum is
    sqrt(max|X_j| * max|W_j|) on both sides, and swapping the operands
    inverts the factor (a transposed or mis-rooted formula fails both)."""
    rng = np.random.default_rng(12)
    ax = (10.0 ** rng.uniform(-2, 3, 512)).astype(np.float32)
    aw = (10.0 ** rng.uniform(-3, 0, 512)).astype(np.float32)
    s = oracle.smooth_factors(ax, aw).astype(np.float64)
    geo = np.sqrt(ax.astype(np.float64) * aw.astype(np.float64))
    np.testing.assert_allclose(ax / s, geo, rtol=1e-6)
    np.testing.assert_allclose(aw * s, geo, rtol=1e-6)
    inv = oracle.smooth_factors(aw, ax).astype(np.float64)
    np.testing.assert_allclose(s * inv, 1.0, rtol=1e-6)
    # floors: a zero weight channel uses 1e-5, and the factor never drops below 1e-5
    f = oracle.smooth_factors(np.array([4.0, 0.0], np.float32), np.array([0.0, 1.0], np.float32))
    assert f[0] == np.float32(2.0) / np.sqrt(np.float32(1e-5)) and f[1] == np.float32(1e-5)


def test_bf16_rounding_helpers(oracle):
    vals = np.array([1.0, 1.00390625, 1.0117188, -3.3e38, 1e-40, np.inf], np.float32)
    bits = f32_to_bf16_bits(vals)
    for v, b in zip(vals, bits):
        assert oracle.lib().kco_f32_to_bf16(float(v)) == int(b)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bits, ref)


# ---------------------------------------------------------------------------
# RMSNorm (tests/test_mamba_ops.cpp:89-101, rmsnorm.cu:40-70)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["rms_basic", "rms_d768", "rms_d4096"])
def test_rmsnorm_reference_kats(oracle, golden, name):
    """The reference C++ tests' recipes (glibc rand) and CPU check: the
    restatement reproduces rmsnorm_cpu's fp32 results bit for bit."""
    y = oracle.rmsnorm(golden[f"{name}_x"], golden[f"{name}_g"], 1e-6)
    np.testing.assert_array_equal(y, golden[f"{name}_expected"])


def test_rmsnorm_reference_kat_python(oracle, golden):
    """test_mamba_bindings.py:251-262 (numpy mean, so another summation
    order): the reference test's own 1e-5 bar."""
    y = oracle.rmsnorm(golden["rms_py_rng3_x"], golden["rms_py_rng3_g"], 1e-6)
    assert np.max(np.abs(y - golden["rms_py_rng3_expected"])) < 1e-5


def test_rmsnorm_closed_forms(oracle):
    # a constant row c: y = g * c / sqrt(c^2 + eps)
    D = 64
    g = np.linspace(0.5, 1.5, D).astype(np.float32)
    x = np.full((3, D), [[2.0], [-0.25], [3.0]], np.float32)
    y = oracle.rmsnorm(x, g, 1e-6)
    c = x[:, :1].astype(np.float64)
    np.testing.assert_allclose(y, g[None, :] * c / np.sqrt(c * c + 1e-6), rtol=2e-7)
    # with g = 1 the output's mean square is ms / (ms + eps): a divisor other
    # than D, or a missing square, moves it
    rng = np.random.default_rng(22)
    x = rng.uniform(-1, 1, (32, 256)).astype(np.float32)
    eps = 0.25
    y = oracle.rmsnorm(x, np.ones(256, np.float32), eps).astype(np.float64)
    ms = np.mean(x.astype(np.float64) ** 2, axis=1)
    np.testing.assert_allclose(np.mean(y * y, axis=1), ms / (ms + eps), rtol=1e-5)


def test_rmsnorm_scale_invariance_exact(oracle):
    """With eps = 0 a power-of-two scale of x cancels exactly (every step
    scales by a power of two), so y is bit-identical."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 300)).astype(np.float32)
    g = rng.uniform(0.5, 2.0, 300).astype(np.float32)
    y = oracle.rmsnorm(x, g, 0.0)
    for k in (-8, 3, 20):
        np.testing.assert_array_equal(oracle.rmsnorm(x * np.float32(2.0 ** k), g, 0.0), y)


def test_rmsnorm_bf16_is_rounded_f32(oracle):
    """bf16 in, bf16 out: the fp32 RMSNorm of the bf16 values, rounded."""
    rng = np.random.default_rng(6)
    xb = f32_to_bf16_bits(rng.standard_normal((5, 4096)).astype(np.float32))
    gb = f32_to_bf16_bits(rng.uniform(0.5, 1.5, 4096).astype(np.float32))
    yb = oracle.rmsnorm(xb, gb, 1e-5)
    ref = oracle.rmsnorm(bf16_bits_to_f32(xb), bf16_bits_to_f32(gb), 1e-5)
    np.testing.assert_array_equal(yb, f32_to_bf16_bits(ref))


# ---------------------------------------------------------------------------
# RMSNorm in the library's fixed summation order, and its FP8 fusion
# ---------------------------------------------------------------------------

def _rn32(fr):
    """A Fraction rounded to the nearest fp32 (ties to even), as np.float32;
    independent of the oracle (exact rational arithmetic)."""
    from fractions import Fraction
    if fr == 0:
        return np.float32(0.0)
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    ulp = Fraction(2) ** (max(e, -126) - 23)
    q = a / ulp
    n = q.numerator // q.denominator
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    v = n * ulp
    if v >= Fraction(2) ** 128:
        return np.float32(sign * np.inf)
    return np.float32(sign * float(v))


def _sumsq_lanes_exact(v: np.ndarray, P: int) -> np.float32:
    """The documented order, restated with exact rationals: lane l takes
    slots l, l + 64, ... of P values, one correctly rounded FMA per element,
    then the xor butterfly with correctly rounded adds."""
    from fractions import Fraction
    D = v.size
    p = []
    for lane in range(64):
        s = Fraction(0)
        for slot in range(lane, (D + P - 1) // P, 64):
            for i in range(slot * P, min(slot * P + P, D)):
                x = Fraction(float(v[i]))
                s = Fraction(float(_rn32(x * x + s)))
        p.append(s)
    for o in (32, 16, 8, 4, 2, 1):
        p = [Fraction(float(_rn32(p[lane] + p[lane ^ o]))) for lane in range(64)]
    return np.float32(float(p[0]))


def _rmsnorm_from_ss(x, g, ss, eps):
    D = x.size
    rms_inv = np.float32(1.0) / np.sqrt(np.float32(ss) / np.float32(D) + np.float32(eps))
    return (g.astype(np.float32) * x.astype(np.float32)) * rms_inv


def test_rn32_helper():
    from fractions import Fraction
    for v in (1.0, -3.5, 1e-40, 3.4e38, 0.1):
        assert _rn32(Fraction(v)) == np.float32(v)
    # a tie between two fp32 neighbours goes to the even one
    one = Fraction(1)
    assert _rn32(one + Fraction(1, 2 ** 24)) == np.float32(1.0)
    assert _rn32(one + Fraction(3, 2 ** 24)) == np.float32(1.0 + 2.0 ** -22)


@pytest.mark.parametrize("D,P", [(4096, 8), (8192, 8), (1000, 8), (4096, 4), (777, 4)])
def test_rmsnorm_lanes_order_exact_restatement(oracle, D, P):
    """kco_rmsnorm_*_lanes against an exact-rational restatement of the
    documented order (FMA per element, lane slots of P values, butterfly):
    bit for bit, on rows whose squares span many binades.  A sequential sum
    (the reference CPU check's order) fails this on these rows."""
    rng = np.random.default_rng(D + P)
    x = (rng.standard_normal(D) * np.exp2(rng.integers(-12, 6, D))).astype(np.float32)
    g = rng.uniform(0.5, 1.5, D).astype(np.float32)
    if P == 8:
        xb, gb = f32_to_bf16_bits(x), f32_to_bf16_bits(g)
        xf, gf = bf16_bits_to_f32(xb), bf16_bits_to_f32(gb)
        ss = _sumsq_lanes_exact(xf, 8)
        want = f32_to_bf16_bits(_rmsnorm_from_ss(xf, gf, ss, 1e-6))
        got = oracle.rmsnorm_lanes(xb[None], gb, 1e-6)[0]
        xs = xf
    else:
        ss = _sumsq_lanes_exact(x, 4)
        want = _rmsnorm_from_ss(x, g, ss, 1e-6)
        got = oracle.rmsnorm_lanes(x[None], g, 1e-6)[0]
        xs = x
    np.testing.assert_array_equal(got, want)
    seq = np.float32(0.0)                     # index order, multiply then add
    for v in xs:
        seq = np.float32(seq + np.float32(v * v))
    assert seq != ss, "test rows do not separate the orders"


def test_rmsnorm_lanes_equals_reference_check_when_sums_are_exact(oracle):
    """With small integer inputs every partial sum of squares is exact in any
    order, so the fixed-order RMSNorm must equal the reference CPU check's
    restatement (pinned bit for bit by the reference KATs) exactly: this pins
    the rest of the formula (D, eps, the square root, the product order)."""
    rng = np.random.default_rng(31)
    for D in (64, 768, 4096, 8192):
        x = rng.integers(-8, 9, (3, D)).astype(np.float32)
        g = rng.uniform(0.5, 1.5, D).astype(np.float32)
        np.testing.assert_array_equal(oracle.rmsnorm_lanes(x, g, 1e-6), oracle.rmsnorm(x, g, 1e-6))
        xb, gb = f32_to_bf16_bits(x), f32_to_bf16_bits(g)
        np.testing.assert_array_equal(oracle.rmsnorm_lanes(xb, gb, 1e-5),
                                      oracle.rmsnorm(xb, gb, 1e-5))


@pytest.mark.parametrize("name,tol", [("rms_basic", 1e-5), ("rms_d768", 1e-4), ("rms_d4096", 1e-4),
                                      ("rms_py_rng3", 1e-5)])
def test_rmsnorm_lanes_within_reference_bars(oracle, golden, name, tol):
    """The reference tests' own bars (test_mamba_ops.cpp:219-300,
    test_mamba_bindings.py:251-262) hold for the fixed order too."""
    y = oracle.rmsnorm_lanes(golden[f"{name}_x"], golden[f"{name}_g"], 1e-6)
    assert np.max(np.abs(y - golden[f"{name}_expected"])) < tol


def test_rmsnorm_quantize_fp8_is_the_composition(oracle):
    """kco_rmsnorm_quantize_fp8_bf16 == per-token FP8 of kco_rmsnorm_bf16_lanes'
    bf16 output, including zero, NaN, infinite and tiny rows."""
    rng = np.random.default_rng(41)
    T, D = 12, 4096
    h = normal_bf16((T, D), seed=42)
    g = f32_to_bf16_bits(rng.uniform(0.5, 1.5, D).astype(np.float32))
    h[1] = 0                                    # all-zero row: scale 1, codes 0
    h[2, 17] = 0x7FC0                           # NaN: the whole row is NaN -> +448
    h[3, 5] = 0x7F80                            # +inf: inf * 0 -> NaN, others +-0
    h[4] = f32_to_bf16_bits(np.full(D, 2.0 ** -70, np.float32))  # tiny row
    h[5, :] = 0x8000                            # -0 row
    q, s = oracle.rmsnorm_quantize_fp8_bf16(h, g, 1e-6)
    y = oracle.rmsnorm_lanes(h, g, 1e-6)
    eq, es = oracle.quantize_fp8_per_token_bf16(y)
    np.testing.assert_array_equal(q, eq)
    np.testing.assert_array_equal(s, es)
    assert s[1] == 1.0 and not q[1].any()
    assert (q[2].view(np.uint8) == 0x7E).all()
    assert (q[5].view(np.uint8) == 0x80).all()


def test_multithreaded_baselines_equal_scalar(oracle):
    """The all-core CPU baselines split rows over threads and compute each
    row exactly as the single-thread loops do."""
    p, s, z = make_int4(515, 1024, 128, seed=51)
    xb = normal_bf16((1024,), seed=52)
    y1 = oracle.gemv_int4_bf16_f32(p, s, z.reshape(-1), xb, 515, 1024, 128)
    for t in (2, 7, 16):
        np.testing.assert_array_equal(
            oracle.gemv_int4_bf16_f32(p, s, z.reshape(-1), xb, 515, 1024, 128, threads=t), y1)
    x, _ = outlier_activations(333, 4096, 0.01, 50.0, seed=53)
    q1, s1 = oracle.quantize_fp8_per_token(x)
    for t in (3, 8):
        q, sc = oracle.quantize_fp8_per_token(x, threads=t)
        np.testing.assert_array_equal(q, q1)
        np.testing.assert_array_equal(sc, s1)


def test_multithreaded_full_size_oracles_equal_scalar(oracle):
    """The row splits the full-size GPU tests use (cfg4's SmoothQuant
    quantizers, cfg3's per-row GEMM) give the single-thread functions' bits:
    every row, with rows not divisible by the thread count, more threads than
    rows, special values (zero rows, NaN, infinity, huge and tiny values) and
    every M of the GEMM's tiles."""
    rng = np.random.default_rng(61)
    for rows, cols in ((37, 1024), (5, 256), (300, 2048)):
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        x[:, rng.choice(cols, 4, replace=False)] *= 100.0
        x[1] = 0.0
        x[2, 3] = np.nan
        x[3, 7] = np.inf
        x[4, :5] = [3e38, -3e38, 1e-38, -1e-40, 6e-8]
        xb = f32_to_bf16_bits(x)
        sm = rng.uniform(0.05, 20.0, cols).astype(np.float32)
        qd1, sd1 = oracle.quantize_fp8_smooth_div(xb, sm)
        qm1, sm1 = oracle.quantize_fp8_smooth_mul_bf16(xb, sm)
        for t in (2, 3, 8, 64):
            qd, sd = oracle.quantize_fp8_smooth_div(xb, sm, threads=t)
            qm, smm = oracle.quantize_fp8_smooth_mul_bf16(xb, sm, threads=t)
            np.testing.assert_array_equal(qd, qd1)
            np.testing.assert_array_equal(sd.view(np.uint32), sd1.view(np.uint32))
            np.testing.assert_array_equal(qm, qm1)
            np.testing.assert_array_equal(smm.view(np.uint32), sm1.view(np.uint32))
    for m, rows, cols, gs in ((1, 37, 256, 128), (5, 100, 512, 64), (17, 33, 1024, 128)):
        p, s, z = make_int4(rows, cols, gs, seed=62 + m)
        xb = normal_bf16((m, cols), seed=63 + m)
        y1 = oracle.gemm_int4_bf16_f64(p, s, z.reshape(-1), xb, m, rows, cols, gs)
        for t in (2, 5, 64):
            y = oracle.gemm_int4_bf16_f64(p, s, z.reshape(-1), xb, m, rows, cols, gs, threads=t)
            np.testing.assert_array_equal(y.view(np.uint64), y1.view(np.uint64))


# ---------------------------------------------------------------------------
# The shuffled INT4 layout (kco_shuffle_int4_mfma)
# ---------------------------------------------------------------------------

def _shuffle_numpy(packed, rows, cols):
    """The layout restated with reshapes: pad rows to 16, view each row as
    [k-block T][kb][16 bytes], reorder to [tile][T][kb][row in tile][16 B]."""
    tiles = (rows + 15) // 16
    p = np.zeros((tiles * 16, cols // 2), np.uint8)
    p[:rows] = packed
    v = p.reshape(tiles, 16, cols // 128, 4, 16)          # tile, i, T, kb, byte
    return v.transpose(0, 2, 3, 1, 4).reshape(-1)          # tile, T, kb, i, byte


@pytest.mark.parametrize("rows,cols", [(16, 128), (1, 128), (33, 256), (100, 1152), (48, 4096)])
def test_shuffle_int4_mfma_layout(oracle, rows, cols):
    rng = np.random.default_rng(rows + cols)
    packed = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    np.testing.assert_array_equal(oracle.shuffle_int4_mfma(packed, rows, cols),
                                  _shuffle_numpy(packed, rows, cols))


@pytest.mark.parametrize("rows,cols", [(32, 256), (21, 384)])
def test_shuffle_int4_mfma_is_a_bijection_of_units(oracle, rows, cols):
    """Tag every 16-byte unit of the input with its index: the output holds
    each index exactly once, and zeros only in the pad rows; unit l of block
    (t, T) comes from row 16 t + l % 16, bytes 64 T + 16 (l // 16)."""
    units = rows * cols // 32
    tags = np.arange(1, units + 1, dtype=np.uint32)
    packed = np.zeros((units, 16), np.uint8)
    packed[:, :4] = tags.view(np.uint8).reshape(units, 4)
    packed = packed.reshape(rows, cols // 2)
    out = oracle.shuffle_int4_mfma(packed, rows, cols).reshape(-1, 16)
    got = out[:, :4].copy().view(np.uint32).reshape(-1)
    assert sorted(got[got != 0].tolist()) == tags.tolist()
    assert (got == 0).sum() == ((rows + 15) // 16 * 16 - rows) * cols // 32
    nT = cols // 128
    for u in range(out.shape[0]):
        t, T, l = u // (64 * nT), (u // 64) % nT, u % 64
        row = 16 * t + l % 16
        want = 0 if row >= rows else row * (cols // 32) + 4 * T + l // 16 + 1
        assert got[u] == want
