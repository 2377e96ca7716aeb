"""ctypes wrapper over the CPU oracle (oracle/kc_oracle.c).

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and
bench.py's ``cpu_baseline`` leg import this module, and only as the checker or
as the timed CPU baseline.  The product path never imports it.

Arrays are numpy; bf16 tensors travel as ``np.uint16`` bit patterns.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libkc_oracle.so"
_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64

_SIGS = {
    "kco_sext4": ([ctypes.c_uint], ctypes.c_int),
    "kco_e4m3_encode": ([ctypes.c_float], ctypes.c_uint8),
    "kco_e4m3_decode": ([ctypes.c_uint8], ctypes.c_float),
    "kco_bf16_to_f32": ([ctypes.c_uint16], ctypes.c_float),
    "kco_f32_to_bf16": ([ctypes.c_float], ctypes.c_uint16),
    "kco_e4m3_sweep_mismatches": ([ctypes.c_uint32, ctypes.c_uint64, _P,
                                   ctypes.POINTER(ctypes.c_uint32)], ctypes.c_uint64),
    "kco_dequantize_int4": ([_P, _P, _P, _P, _I64, _I64, _I64], None),
    "kco_shuffle_int4_mfma": ([_P, _P, _I64, _I64], None),
    "kco_gemv_int4_f64": ([_P, _P, _P, _P, _P, _I64, _I64, _I64], None),
    "kco_gemv_int4_refkernel_f32": ([_P, _P, _P, _P, _P, _I64, _I64, _I64], None),
    "kco_gemm_int4_bf16_f64": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64], None),
    "kco_gemv_int4_bf16_f32": ([_P, _P, _P, _P, _P, _I64, _I64, _I64], None),
    "kco_quantize_fp8_per_token": ([_P, _P, _P, _I64, _I64], None),
    "kco_quantize_fp8_per_tensor": ([_P, _P, ctypes.c_float, _I64], None),
    "kco_dequantize_fp8": ([_P, _P, _P, _I64, _I64, ctypes.c_int], None),
    "kco_smoothquant_scale": ([_P, _P, _P, _I64, _I64], None),
    "kco_quantize_fp8_per_token_bf16": ([_P, _P, _P, _I64, _I64], None),
    "kco_col_absmax_f32": ([_P, _P, _I64, _I64], None),
    "kco_col_absmax_bf16": ([_P, _P, _I64, _I64], None),
    "kco_smooth_factors": ([_P, _P, _P, _I64], None),
    "kco_quantize_fp8_smooth_div_f32": ([_P, _P, _P, _P, _I64, _I64], None),
    "kco_quantize_fp8_smooth_div_bf16": ([_P, _P, _P, _P, _I64, _I64], None),
    "kco_quantize_fp8_smooth_mul_bf16": ([_P, _P, _P, _P, _I64, _I64], None),
    "kco_rmsnorm_f32": ([_P, _P, _P, _I64, _I64, ctypes.c_float], None),
    "kco_rmsnorm_bf16": ([_P, _P, _P, _I64, _I64, ctypes.c_float], None),
    "kco_gemv_int4_bf16_f32_mt": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, ctypes.c_int], None),
    "kco_quantize_fp8_per_token_mt": ([_P, _P, _P, _I64, _I64, ctypes.c_int], None),
    "kco_quantize_fp8_smooth_div_bf16_mt": ([_P, _P, _P, _P, _I64, _I64, ctypes.c_int], None),
    "kco_quantize_fp8_smooth_mul_bf16_mt": ([_P, _P, _P, _P, _I64, _I64, ctypes.c_int], None),
    "kco_gemm_int4_bf16_f64_mt": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, ctypes.c_int],
                                  None),
    "kco_rmsnorm_f32_lanes": ([_P, _P, _P, _I64, _I64, ctypes.c_float], None),
    "kco_rmsnorm_bf16_lanes": ([_P, _P, _P, _I64, _I64, ctypes.c_float, _P], None),
    "kco_rmsnorm_quantize_fp8_bf16": ([_P, _P, ctypes.c_float, _P, _P, _I64, _I64, _P, _P],
                                      None),
}


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise FileNotFoundError(
                f"{_LIB_PATH} missing: build it with `make -C oracle`")
        _lib = ctypes.CDLL(str(_LIB_PATH))
        for name, (argtypes, restype) in _SIGS.items():
            fn = getattr(_lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
    return _lib


def _p(a: np.ndarray) -> ctypes.c_void_p:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return ctypes.c_void_p(a.ctypes.data)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ---- scalar helpers -------------------------------------------------------

def sext4(n: int) -> int:
    return lib().kco_sext4(n)


def e4m3_encode(x: float) -> int:
    return int(lib().kco_e4m3_encode(x))


def e4m3_decode_table() -> np.ndarray:
    return np.array([lib().kco_e4m3_decode(c) for c in range(256)], dtype=np.float32)


def sweep_mismatches(start: int, codes: np.ndarray):
    """(mismatch count, first bad fp32 bit pattern) for clamp+encode."""
    codes = _c(codes, np.uint8)
    first = ctypes.c_uint32(0)
    bad = lib().kco_e4m3_sweep_mismatches(start, codes.size, _p(codes),
                                          ctypes.byref(first))
    return int(bad), int(first.value)


# ---- INT4 -----------------------------------------------------------------

def dequantize_int4(packed, scales, zeros, rows, cols, group_size):
    packed, scales, zeros = _c(packed, np.uint8), _c(scales, np.float32), _c(zeros, np.uint8)
    out = np.empty((rows, cols), np.float32)
    lib().kco_dequantize_int4(_p(packed), _p(scales), _p(zeros), _p(out),
                              rows, cols, group_size)
    return out


def shuffle_int4_mfma(packed, rows, cols):
    """The matrix-core GEMMs' shuffled layout of packed [rows, cols/2]:
    [ceil(rows/16)*16 * cols/2] bytes (kco_shuffle_int4_mfma)."""
    packed = _c(packed, np.uint8)
    out = np.empty(((rows + 15) // 16) * 16 * (cols // 2), np.uint8)
    lib().kco_shuffle_int4_mfma(_p(packed), _p(out), rows, cols)
    return out


def gemv_int4_f64(packed, scales, zeros, x, rows, cols, group_size):
    packed, scales, zeros = _c(packed, np.uint8), _c(scales, np.float32), _c(zeros, np.uint8)
    x = _c(x, np.float32)
    y = np.empty(rows, np.float64)
    lib().kco_gemv_int4_f64(_p(packed), _p(scales), _p(zeros), _p(x), _p(y),
                            rows, cols, group_size)
    return y


def gemv_int4_refkernel_f32(packed, scales, zeros, x, rows, cols, group_size):
    packed, scales, zeros = _c(packed, np.uint8), _c(scales, np.float32), _c(zeros, np.uint8)
    x = _c(x, np.float32)
    y = np.empty(rows, np.float32)
    lib().kco_gemv_int4_refkernel_f32(_p(packed), _p(scales), _p(zeros), _p(x),
                                      _p(y), rows, cols, group_size)
    return y


def gemm_int4_bf16_f64(packed, scales, zeros, x_bf16, m, rows, cols, group_size, threads=1):
    """Reference GEMV applied to each of the m bf16 activation rows -> [m, rows];
    threads > 1 splits the rows over that many OpenMP threads (same sums)."""
    packed, scales, zeros = _c(packed, np.uint8), _c(scales, np.float32), _c(zeros, np.uint8)
    x_bf16 = _c(x_bf16, np.uint16)
    y = np.empty((m, rows), np.float64)
    fn = lib().kco_gemm_int4_bf16_f64_mt if threads > 1 else lib().kco_gemm_int4_bf16_f64
    args = (_p(packed), _p(scales), _p(zeros), _p(x_bf16), _p(y), m, rows, cols, group_size)
    fn(*args, int(threads)) if threads > 1 else fn(*args)
    return y


def gemv_int4_bf16_f32(packed, scales, zeros, x_bf16, rows, cols, group_size, threads=1):
    """The scalar CPU GEMV (fp32 accumulation in index order); threads > 1
    splits its rows over that many OpenMP threads (same results)."""
    packed, scales, zeros = _c(packed, np.uint8), _c(scales, np.float32), _c(zeros, np.uint8)
    x_bf16 = _c(x_bf16, np.uint16)
    y = np.empty(rows, np.float32)
    if threads > 1:
        lib().kco_gemv_int4_bf16_f32_mt(_p(packed), _p(scales), _p(zeros), _p(x_bf16),
                                        _p(y), rows, cols, group_size, int(threads))
    else:
        lib().kco_gemv_int4_bf16_f32(_p(packed), _p(scales), _p(zeros), _p(x_bf16),
                                     _p(y), rows, cols, group_size)
    return y


# ---- FP8 ------------------------------------------------------------------

def quantize_fp8_per_token(x, threads=1):
    x = _c(x, np.float32)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    if threads > 1:
        lib().kco_quantize_fp8_per_token_mt(_p(x), _p(q), _p(s), rows, cols, int(threads))
    else:
        lib().kco_quantize_fp8_per_token(_p(x), _p(q), _p(s), rows, cols)
    return q, s


def quantize_fp8_per_tensor(x, scale):
    x = _c(x, np.float32)
    q = np.empty(x.shape, np.int8)
    lib().kco_quantize_fp8_per_tensor(_p(x), _p(q), float(scale), x.size)
    return q


def dequantize_fp8(q, scales, rows, cols, per_token=True):
    q, scales = _c(q, np.int8), _c(scales, np.float32)
    out = np.empty((rows, cols), np.float32)
    lib().kco_dequantize_fp8(_p(q), _p(scales), _p(out), rows, cols, int(per_token))
    return out


def smoothquant_scale(x, smooth):
    x, smooth = _c(x, np.float32), _c(smooth, np.float32)
    rows, cols = x.shape
    out = np.empty_like(x)
    lib().kco_smoothquant_scale(_p(x), _p(smooth), _p(out), rows, cols)
    return out


def quantize_fp8_per_token_bf16(x_bf16):
    x_bf16 = _c(x_bf16, np.uint16)
    rows, cols = x_bf16.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    lib().kco_quantize_fp8_per_token_bf16(_p(x_bf16), _p(q), _p(s), rows, cols)
    return q, s


def rmsnorm(x, g, eps=1e-6):
    """RMSNorm of every row of x (tests/test_mamba_ops.cpp:89-101): fp32 x, g
    give fp32 y; bf16 bit patterns (uint16) give bf16 bits."""
    if np.asarray(x).dtype == np.uint16:
        x, g = _c(x, np.uint16), _c(g, np.uint16)
        fn = lib().kco_rmsnorm_bf16
    else:
        x, g = _c(x, np.float32), _c(g, np.float32)
        fn = lib().kco_rmsnorm_f32
    x2 = x.reshape(-1, x.shape[-1])
    y = np.empty_like(x2)
    fn(_p(x2), _p(g), _p(y), x2.shape[0], x2.shape[1], float(eps))
    return y.reshape(x.shape)


def rmsnorm_lanes(x, g, eps=1e-6):
    """RMSNorm with the sum of squares in the library's fixed lane order
    (launch_rmsnorm / kc_rmsnorm_bf16): fp32 in, fp32 out; bf16 bit patterns
    (uint16) in, bf16 bits out."""
    if np.asarray(x).dtype == np.uint16:
        x, g = _c(x, np.uint16), _c(g, np.uint16)
        x2 = x.reshape(-1, x.shape[-1])
        y = np.empty_like(x2)
        tmp = np.empty(x2.shape[1], np.float32)
        lib().kco_rmsnorm_bf16_lanes(_p(x2), _p(g), _p(y), x2.shape[0], x2.shape[1],
                                     float(eps), _p(tmp))
    else:
        x, g = _c(x, np.float32), _c(g, np.float32)
        x2 = x.reshape(-1, x.shape[-1])
        y = np.empty_like(x2)
        lib().kco_rmsnorm_f32_lanes(_p(x2), _p(g), _p(y), x2.shape[0], x2.shape[1],
                                    float(eps))
    return y.reshape(x.shape)


def rmsnorm_quantize_fp8_bf16(h_bf16, g_bf16, eps=1e-6):
    """(codes int8 [T, D], scales fp32 [T]) of rmsnorm_lanes(h, g) (bf16)
    quantized per token, computed row by row in C."""
    h_bf16, g_bf16 = _c(h_bf16, np.uint16), _c(g_bf16, np.uint16)
    T, D = h_bf16.shape
    q = np.empty((T, D), np.int8)
    s = np.empty(T, np.float32)
    tmp = np.empty(max(D, 1), np.float32)
    ytmp = np.empty(max(D, 1), np.uint16)
    lib().kco_rmsnorm_quantize_fp8_bf16(_p(h_bf16), _p(g_bf16), float(eps), _p(q), _p(s), T, D,
                                        _p(tmp), _p(ytmp))
    return q, s


def col_absmax(x):
    if x.dtype == np.uint16:
        x = _c(x, np.uint16)
        fn = lib().kco_col_absmax_bf16
    else:
        x = _c(x, np.float32)
        fn = lib().kco_col_absmax_f32
    rows, cols = x.shape
    out = np.empty(cols, np.float32)
    fn(_p(x), _p(out), rows, cols)
    return out


def smooth_factors(amax_x, amax_w):
    amax_x, amax_w = _c(amax_x, np.float32), _c(amax_w, np.float32)
    s = np.empty_like(amax_x)
    lib().kco_smooth_factors(_p(amax_x), _p(amax_w), _p(s), amax_x.size)
    return s


def quantize_fp8_smooth_div(x, s, threads=1):
    """x [rows, cols] fp32 or bf16 bits; returns (codes, scales) of (x / s);
    threads > 1 (bf16 x) splits the rows over that many OpenMP threads."""
    s = _c(s, np.float32)
    mt = False
    if x.dtype == np.uint16:
        x = _c(x, np.uint16)
        mt = threads > 1
        fn = lib().kco_quantize_fp8_smooth_div_bf16_mt if mt else lib().kco_quantize_fp8_smooth_div_bf16
    else:
        x = _c(x, np.float32)
        fn = lib().kco_quantize_fp8_smooth_div_f32
    rows, cols = x.shape
    q = np.empty((rows, cols), np.int8)
    sc = np.empty(rows, np.float32)
    args = (_p(x), _p(s), _p(q), _p(sc), rows, cols)
    fn(*args, int(threads)) if mt else fn(*args)
    return q, sc


def quantize_fp8_smooth_mul_bf16(w_bf16, s, threads=1):
    w_bf16, s = _c(w_bf16, np.uint16), _c(s, np.float32)
    rows, cols = w_bf16.shape
    q = np.empty((rows, cols), np.int8)
    sc = np.empty(rows, np.float32)
    args = (_p(w_bf16), _p(s), _p(q), _p(sc), rows, cols)
    if threads > 1:
        lib().kco_quantize_fp8_smooth_mul_bf16_mt(*args, int(threads))
    else:
        lib().kco_quantize_fp8_smooth_mul_bf16(*args)
    return q, sc


def lib_path() -> str:
    return os.fspath(_LIB_PATH)


# ---- GPTQ / AWQ checkpoint formats ------------------------------------------
# Restated from the published packing of AutoGPTQ 0.7 and AutoAWQ 0.2 (the
# reference ships no converter; it calls its own layout "GPTQ/AWQ-style",
# quant_int4.cu:5).  Both dequantize as W[k, n] = (u - zu) * s with unsigned
# nibbles u, zu in 0..15 (GPTQ's original format stores zu - 1).

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)  # nibble i of a word holds column 8c + AWQ_ORDER[i]


def _nibbles(words):
    w = np.ascontiguousarray(words).view(np.uint32)
    return ((w[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).astype(np.uint8)


def gptq_unpack(qweight, qzeros, zero_offset=1):
    """qweight int32 [K/8, N], qzeros int32 [G, N/8] -> u [K, N], zu [G, N]."""
    u = _nibbles(qweight)                      # [K/8, N, 8]: nibble i = k 8r + i
    u = u.transpose(0, 2, 1).reshape(-1, u.shape[1])
    z = _nibbles(qzeros).reshape(qzeros.shape[0], -1).astype(np.int32) + zero_offset
    return u, z


def gptq_pack(u, zu, zero_offset=1):
    """Inverse of gptq_unpack (zu - zero_offset must fit a nibble)."""
    K, N = u.shape
    uu = u.astype(np.uint32).reshape(K // 8, 8, N)
    qweight = np.zeros((K // 8, N), np.uint32)
    for i in range(8):
        qweight |= uu[:, i, :] << np.uint32(4 * i)
    zs = (zu - zero_offset).astype(np.int64)
    assert zs.min() >= 0 and zs.max() <= 15
    zz = zs.astype(np.uint32).reshape(zu.shape[0], N // 8, 8)
    qzeros = np.zeros((zu.shape[0], N // 8), np.uint32)
    for i in range(8):
        qzeros |= zz[:, :, i] << np.uint32(4 * i)
    return qweight.view(np.int32), qzeros.view(np.int32)


def awq_unpack(qweight, qzeros):
    """qweight int32 [K, N/8], qzeros int32 [G, N/8] -> u [K, N], zu [G, N]."""
    def cols(words):
        nib = _nibbles(words)                  # [R, N/8, 8]: nibble i -> column 8c + order[i]
        out = np.empty_like(nib)
        out[:, :, list(AWQ_ORDER)] = nib
        return out.reshape(words.shape[0], -1)
    return cols(qweight), cols(qzeros).astype(np.int32)


def awq_pack(u, zu):
    def words(vals):
        R, N = vals.shape
        v = vals.astype(np.uint32).reshape(R, N // 8, 8)
        w = np.zeros((R, N // 8), np.uint32)
        for i in range(8):
            w |= v[:, :, AWQ_ORDER[i]] << np.uint32(4 * i)
        return w.view(np.int32)
    return words(u), words(zu)


def int4_source_dequant(u, zu, scales16, g_idx=None, group_size=128):
    """W [K, N] fp32 = (u - zu[g(k)]) * s[g(k)], one fp32 rounding."""
    K = u.shape[0]
    g = np.arange(K) // group_size if g_idx is None else np.asarray(g_idx)
    s = np.asarray(scales16, np.float16).astype(np.float32)
    d = (u.astype(np.int32) - zu[g]).astype(np.float32)
    return d * s[g]


def convert_to_reference(u, zu, scales16, perm=None, group_size=128):
    """Reference layout (packed [N, K/2], scales [N, G] fp32, zeros [N, G/2])
    of a source checkpoint: output column j takes input k = perm[j].  Groups
    with zu >= 8 store q = u - 8, z = zu - 8, s; the others q = 7 - u,
    z = 7 - zu, -s (exact: the integer difference is kept, the scale negated)."""
    K, N = u.shape
    kk = np.arange(K) if perm is None else np.asarray(perm)
    uo = u[kk].T.astype(np.int32)                                 # [N, K]
    zt = zu.T                                                     # [N, G]
    up = zt >= 8
    upk = np.repeat(up, group_size, axis=1)                       # [N, K]
    q = np.where(upk, uo - 8, 7 - uo) & 0xF
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    z = np.where(up, zt - 8, 7 - zt).astype(np.uint8)
    zeros = (z[:, 0::2] | (z[:, 1::2] << 4)).astype(np.uint8)
    s = np.asarray(scales16, np.float16).astype(np.float32).T
    scales = np.where(up, s, -s).astype(np.float32)
    return packed, np.ascontiguousarray(scales), zeros


# ---- FP8 W8A8 GEMM ----------------------------------------------------------

def gemm_fp8_w8a8_f64(qx, sx, qw, sw):
    """Y[m, n] = sx[m] sw[n] sum_k e4m3(qx[m, k]) e4m3(qw[n, k]) in fp64.

    The reference's FP8 GEMM is the product of the dequantized codes with the
    per-row scales applied to the result (examples/python/transformer/
    fp8_quant.py:55-60: quantize W and x, multiply, dequantize with the
    combined scales); here the codes decode through kco_e4m3_decode
    (fp8_quant.cu's E4M3 format), qx [M, K] per-token, qw [N, K] per-channel."""
    table = e4m3_decode_table().astype(np.float64)
    a = table[np.ascontiguousarray(qx).view(np.uint8)]
    b = table[np.ascontiguousarray(qw).view(np.uint8)]
    return (a @ b.T) * np.asarray(sx, np.float64)[:, None] * np.asarray(sw, np.float64)[None, :]
