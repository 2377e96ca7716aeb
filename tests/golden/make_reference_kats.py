"""Regenerate tests/golden/reference_kats.npz.

Each fixture reproduces one known-answer test of the reference's own test
suite: the same inputs (glibc ``srand``/``rand`` through ctypes for the C++
tests, numpy ``default_rng`` for the Python tests) and the expected values the
reference test computes for them, by the expression that test uses.  Nothing
here imports or runs reference code; the input recipes and expected-value
expressions are restated from the cited lines.

    python tests/golden/make_reference_kats.py
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

OUT = Path(__file__).with_name("reference_kats.npz")
_libc = ctypes.CDLL("libc.so.6")
_libc.rand.restype = ctypes.c_int
RAND_MAX = 2147483647  # glibc


def c_rand_unit_f32() -> np.float32:
    """((float)rand() / RAND_MAX): int -> float, then an fp32 divide."""
    return np.float32(np.float32(_libc.rand()) / np.float32(RAND_MAX))


def c_fill_rand(n: int, lo: float, hi: float) -> np.ndarray:
    """tests/test_mamba_ops.cpp:31-33: lo + (hi - lo) * (float)rand() / RAND_MAX,
    left to right in fp32."""
    lo32, span = np.float32(lo), np.float32(np.float32(hi) - np.float32(lo))
    return np.array([lo32 + (span * np.float32(_libc.rand())) / np.float32(RAND_MAX)
                     for _ in range(n)], np.float32)


def rmsnorm_cpu(x: np.ndarray, g: np.ndarray, eps: np.float32) -> np.ndarray:
    """tests/test_mamba_ops.cpp:89-101: ss += x*x in index order (fp32),
    rms_inv = 1 / sqrt(ss / D + eps), y = g * x * rms_inv."""
    rows, D = x.shape
    ss = np.zeros(rows, np.float32)
    for i in range(D):
        ss = (ss + x[:, i] * x[:, i]).astype(np.float32)
    rms_inv = np.float32(1.0) / np.sqrt(ss / np.float32(D) + eps)
    return (g[None, :] * x * rms_inv[:, None]).astype(np.float32)


def pack_nibbles(w: np.ndarray) -> np.ndarray:
    """tests/test_quant_int4.cpp:31-33: low nibble = even column."""
    w = w.astype(np.int64)
    lo = w[:, 0::2] & 0xF
    hi = w[:, 1::2] & 0xF
    return (lo | (hi << 4)).astype(np.uint8)


def main() -> None:
    fx: dict[str, np.ndarray] = {}

    # tests/test_quant_int4.cpp:35-88 (4x8, gs 8, (i%16)-8, scale 0.125, zp 0)
    rows, cols, gs = 4, 8, 8
    w = ((np.arange(rows * cols) % 16) - 8).astype(np.int8).reshape(rows, cols)
    fx["deq_basic_packed"] = pack_nibbles(w)
    fx["deq_basic_scales"] = np.full((rows, cols // gs), 0.125, np.float32)
    fx["deq_basic_zeros"] = np.zeros((rows, 1), np.uint8)  # zeros_cols = sc/2 + sc%2
    fx["deq_basic_expected"] = w.astype(np.float32) * np.float32(0.125)
    fx["deq_basic_shape"] = np.array([rows, cols, gs])

    # tests/test_quant_int4.cpp:90-146 (16x16, gs 8, srand(42), rand()%15-7,
    # scale 0.1, x = rand()/RAND_MAX*2-1, y_ref fp32 loop :117-121, tol 1e-4)
    rows, cols, gs = 16, 16, 8
    _libc.srand(42)
    w = np.array([(_libc.rand() % 15) - 7 for _ in range(rows * cols)],
                 np.int8).reshape(rows, cols)
    x = np.array([c_rand_unit_f32() * np.float32(2.0) - np.float32(1.0)
                  for _ in range(cols)], np.float32)
    s = np.float32(0.1)
    y = np.zeros(rows, np.float32)
    for r in range(rows):
        for c in range(cols):
            y[r] = np.float32(y[r] + np.float32(np.float32(w[r, c]) * s) * x[c])
    sc = cols // gs
    fx["gemv_srand42_packed"] = pack_nibbles(w)
    fx["gemv_srand42_scales"] = np.full((rows, sc), s, np.float32)
    fx["gemv_srand42_zeros"] = np.zeros((rows, sc // 2 + sc % 2), np.uint8)
    fx["gemv_srand42_x"] = x
    fx["gemv_srand42_expected"] = y
    fx["gemv_srand42_shape"] = np.array([rows, cols, gs])

    # tests/test_quant_int4.cpp:148-199 (4x128, gs 64, srand(13),
    # scales 0.05 + 0.01*i, expected (float)w * scale, tol 1e-5)
    rows, cols, gs = 4, 128, 64
    _libc.srand(13)
    w = np.array([(_libc.rand() % 15) - 7 for _ in range(rows * cols)],
                 np.int8).reshape(rows, cols)
    sc = cols // gs
    scales = np.array([np.float32(0.05) + np.float32(0.01) * np.float32(i)
                       for i in range(rows * sc)], np.float32).reshape(rows, sc)
    exp = np.empty((rows, cols), np.float32)
    for r in range(rows):
        for c in range(cols):
            exp[r, c] = np.float32(w[r, c]) * scales[r, c // gs]
    fx["deq_multigroup_packed"] = pack_nibbles(w)
    fx["deq_multigroup_scales"] = scales
    fx["deq_multigroup_zeros"] = np.zeros((rows, sc // 2 + sc % 2), np.uint8)
    fx["deq_multigroup_expected"] = exp
    fx["deq_multigroup_shape"] = np.array([rows, cols, gs])

    # src/python/tests/test_transformer_bindings.py:185-196
    rows, cols, gs = 4, 16, 8
    rng = np.random.default_rng(42)
    w = rng.integers(-7, 8, (rows, cols), dtype=np.int8)
    sc = cols // gs
    fx["deq_rng42_packed"] = pack_nibbles(w)
    fx["deq_rng42_scales"] = np.full((rows, sc), 0.125, np.float32)
    fx["deq_rng42_zeros"] = np.zeros((rows, sc // 2 + sc % 2), np.uint8)
    fx["deq_rng42_expected"] = w.astype(np.float32) * np.float32(0.125)
    fx["deq_rng42_shape"] = np.array([rows, cols, gs])

    # src/python/tests/test_triton_kernels.py:98-119 (_make_int4_data) and the
    # numpy reference :76-95 (fp32 W, then W @ x); cases :244-256
    for name, (rows, cols, gs, seed) in {
        "triton_small": (4, 256, 128, 0),
        "triton_medium": (64, 1024, 128, 7),
        "triton_gs64": (8, 512, 64, 3),
    }.items():
        rng = np.random.default_rng(seed)
        G = cols // gs
        nzb = (G + 1) // 2
        w_int4 = rng.integers(-8, 8, size=(rows, cols), dtype=np.int8)
        packed = pack_nibbles(w_int4)
        scales = rng.uniform(0.01, 0.1, (rows, G)).astype(np.float32)
        zeros = np.zeros((rows, nzb), np.uint8)
        x = rng.uniform(-1.0, 1.0, cols).astype(np.float32)
        W = np.empty((rows, cols), np.float32)
        for r in range(rows):
            for c in range(cols):
                W[r, c] = np.float32(w_int4[r, c]) * scales[r, c // gs]
        fx[f"{name}_packed"] = packed
        fx[f"{name}_scales"] = scales
        fx[f"{name}_zeros"] = zeros
        fx[f"{name}_x"] = x
        fx[f"{name}_expected"] = (W @ x).astype(np.float32)
        fx[f"{name}_shape"] = np.array([rows, cols, gs])

    # tests/test_fp8_quant.cpp:34-71 (8x64, srand(42), rand()/RAND_MAX*2-1)
    _libc.srand(42)
    fx["fp8_tok_srand42_x"] = np.array(
        [c_rand_unit_f32() * np.float32(2.0) - np.float32(1.0) for _ in range(8 * 64)],
        np.float32).reshape(8, 64)
    # tests/test_fp8_quant.cpp:137-174 (4x32, srand(7), *4-2, scale absmax/448)
    _libc.srand(7)
    xt = np.array([c_rand_unit_f32() * np.float32(4.0) - np.float32(2.0)
                   for _ in range(4 * 32)], np.float32).reshape(4, 32)
    fx["fp8_tensor_srand7_x"] = xt
    fx["fp8_tensor_srand7_scale"] = np.array(
        [np.float32(np.abs(xt).max()) / np.float32(448.0)], np.float32)
    # tests/test_fp8_quant.cpp:99-135 (4x16 ones, column 0 = 100, s[0] = 100)
    xs = np.ones((4, 16), np.float32)
    xs[:, 0] = 100.0
    ss = np.ones(16, np.float32)
    ss[0] = 100.0
    fx["smooth_kat_x"] = xs
    fx["smooth_kat_s"] = ss
    fx["smooth_kat_expected"] = np.ones((4, 16), np.float32)
    # test_transformer_bindings.py:212-220 and test_vllm_backend.py:214-223
    fx["fp8_tok_rng42_x"] = np.random.default_rng(42).uniform(-1, 1, (8, 64)).astype(np.float32)
    fx["fp8_tok_rng11_x"] = np.random.default_rng(11).uniform(-1, 1, (8, 64)).astype(np.float32)

    # RMSNorm, tests/test_mamba_ops.cpp:219-300: fill_rand (:31-33) from
    # glibc srand/rand, expected values by rmsnorm_cpu (:89-101), tolerances
    # 1e-5 / 1e-4 / 1e-4 max abs.  Only the leading rows of the larger cases
    # are kept (their rows come from the full recipe).
    for name, seed, rows, D, xr, gr, keep in (("rms_basic", 3, 8, 8, (-1, 1), (0.5, 1.5), 8),
                                              ("rms_d768", 77, 128, 768, (-2, 2), (0.8, 1.2), 4),
                                              ("rms_d4096", 13, 16, 4096, (-1, 1), (0.9, 1.1), 2)):
        _libc.srand(seed)
        x = c_fill_rand(rows * D, *xr).reshape(rows, D)
        g = c_fill_rand(D, *gr)
        fx[f"{name}_x"] = x[:keep]
        fx[f"{name}_g"] = g
        fx[f"{name}_expected"] = rmsnorm_cpu(x[:keep], g, np.float32(1e-6))

    # RMSNorm, src/python/tests/test_mamba_bindings.py:251-262 (default_rng(3),
    # expected by rmsnorm_ref :100-113 in float32 numpy, tol 1e-5)
    rng = np.random.default_rng(3)
    x = rng.uniform(-1, 1, (8, 64)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 64).astype(np.float32)
    ss = np.mean(x ** 2, axis=-1, keepdims=True)
    fx["rms_py_rng3_x"] = x
    fx["rms_py_rng3_g"] = g
    fx["rms_py_rng3_expected"] = (g * x * (1.0 / np.sqrt(ss + 1e-6))).astype(np.float32)

    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT} ({len(fx)} arrays)")


if __name__ == "__main__":
    main()
