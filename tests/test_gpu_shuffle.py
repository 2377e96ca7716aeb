"""The shuffled INT4 layout of the matrix-core kernels (kc_shuffle_int4_mfma,
kc_gemm_int4_bf16_shuffled): the weight-format bridge's optional
"MFMA-friendly" layout.  Bars: the conversion bit for bit against the oracle
(kco_shuffle_int4_mfma, itself pinned in test_oracle.py); where both layouts
run the same kernel (m >= 9, and m 2..8 with K a multiple of 1024 up to
12288, where the reference layout takes the K-split kernel's pair form) the
GEMM on the shuffled layout bit for bit against kc_gemm_int4_bf16 on the
reference layout (the same arithmetic, other addresses); for the other
m 2..8 shapes (the K-split kernel on the shuffled layout, the X-resident
kernel on the reference layout: other summation orders) and m == 1 (a
matrix-core GEMV of its own) within the bf16 tolerance of the fp64 oracle, as
the other bf16 GEMM and GEMV tests."""
import ctypes

import numpy as np
import pytest

import kc_abi
from kc_abi import ptr, stream
from kc_data import bf16_bits_to_f32, make_int4, normal_bf16, rel_l2

pytestmark = pytest.mark.gpu

KC_ERR_INVALID_ARGUMENT = 1


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _dev_bf16(torch, bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


def _host_bf16(t):
    return bf16_bits_to_f32(t.view(__import__("torch").int16).cpu().numpy().view(np.uint16))


def _lib():
    L = kc_abi.lib()
    L.kc_shuffled_int4_bytes.restype = ctypes.c_int64
    L.kc_shuffled_int4_bytes.argtypes = [ctypes.c_int64, ctypes.c_int64]
    return L


def _shuffle(torch, dp, rows, cols):
    L = _lib()
    nbytes = L.kc_shuffled_int4_bytes(rows, cols)
    assert nbytes == (rows + 15) // 16 * 16 * cols // 2
    out = torch.full((nbytes,), 0xA5, dtype=torch.uint8, device="cuda")
    print(f"kc_shuffle_int4_mfma rows={rows} cols={cols}", flush=True)
    kc_abi.check("kc_shuffle_int4_mfma", L.kc_shuffle_int4_mfma(ptr(dp), ptr(out), rows, cols, stream()))
    return out


def _gemm(torch, fn, dp, ds, dz, dx, m, rows, cols, gs):
    dy = torch.full((m, rows), float("nan"), dtype=torch.bfloat16, device="cuda")
    print(f"{fn} m={m} rows={rows} cols={cols} gs={gs}", flush=True)
    st = getattr(_lib(), fn)(ptr(dp), ptr(ds), ptr(dz), ptr(dx), ptr(dy), m, rows, cols, gs, stream())
    kc_abi.check(fn, st)
    torch.cuda.synchronize()
    return dy


@pytest.mark.parametrize("rows,cols", [(16, 128), (33, 256), (1000, 1024), (4096, 4096),
                                       (7, 1152), (6144, 14336)])
def test_shuffle_matches_oracle(gpu, oracle, rows, cols):
    torch = gpu
    packed, _, _ = make_int4(rows, cols, 128, seed=rows + cols)
    out = _shuffle(torch, _dev(torch, packed), rows, cols)
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.shuffle_int4_mfma(packed, rows, cols))


# the reference-layout GEMM's shape list (tests/test_gpu_int4.py), every path:
# X resident (one to four phases), K-split, the chunked and the four-tile
# fallbacks, ragged row tiles, spare waves, group sizes 128..512
GEMM_SHAPES = [(3, 64, 256, 128), (17, 130, 2048, 256), (33, 48, 640, 128), (64, 16, 128, 128),
               (2, 250, 384, 128), (4, 1000, 1280, 256), (3, 4096, 4096, 128),
               (4, 7 * 16 * 3 + 5, 2048, 512), (4, 33, 32768, 128), (16, 48, 1024, 128),
               (8, 300, 4096, 128), (12, 257, 2048, 256), (16, 100, 8192, 128),
               (6, 7 * 16 + 1, 8192, 512), (8, 500, 8192, 128), (12, 100, 24576, 128),
               (9, 40, 2048, 256), (33, 70, 1024, 128), (64, 7 * 16 * 2 + 9, 2048, 256),
               (48, 200, 8192, 128), (20, 224, 4096, 128), (32, 1000, 4096, 128),
               (40, 113, 16384, 128), (17, 7, 256, 256), (63, 1, 512, 128), (26, 130, 1152, 128),
               (40, 200, 4096, 512), (64, 50, 24576, 128), (4, 28672, 8192, 128),
               (16, 28672, 8192, 128), (64, 28672, 8192, 128),
               # the reference layout's pair form: one and three pairs per wave,
               # K at its limit for M <= 16; past its limit for M <= 32
               (3, 200, 1024, 128), (2, 77, 3072, 256), (8, 130, 12288, 128),
               (20, 60, 10240, 128)]


def same_kernels(m, cols):
    """Whether both layouts run the same GEMM kernel: the K-split kernel from
    m = 9, and from m = 2 where the reference layout takes its pair form (K a
    multiple of 1024, up to 12288); other m 2..8 shapes run the X-resident
    kernel on the reference layout."""
    return m >= 9 or (m >= 2 and cols % 1024 == 0 and cols <= 12288)


@pytest.mark.parametrize("m,rows,cols,gs", GEMM_SHAPES)
def test_gemm_shuffled_equals_reference_layout(gpu, oracle, m, rows, cols, gs):
    torch = gpu
    packed, scales, zeros = make_int4(rows, cols, gs, seed=m * 1000 + rows)
    xb = normal_bf16((m, cols), seed=m + rows)
    dp, ds, dz, dx = _dev(torch, packed), _dev(torch, scales), _dev(torch, zeros), _dev_bf16(torch, xb)
    ref = _gemm(torch, "kc_gemm_int4_bf16", dp, ds, dz, dx, m, rows, cols, gs)
    sh = _shuffle(torch, dp, rows, cols)
    y = _gemm(torch, "kc_gemm_int4_bf16_shuffled", sh, ds, dz, dx, m, rows, cols, gs)
    if same_kernels(m, cols):
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
    else:
        truth = oracle.gemm_int4_bf16_f64(packed, scales, zeros.reshape(-1), xb, m, rows, cols, gs,
                                          threads=16)
        assert np.all(np.isfinite(_host_bf16(y)))
        assert rel_l2(_host_bf16(y), truth) < 3e-3
        assert rel_l2(_host_bf16(ref), truth) < 3e-3


@pytest.mark.parametrize("rows,cols,gs", [(6144, 4096, 128), (4096, 4096, 128), (28672, 4096, 128),
                                          (4096, 14336, 128),
                                          # K 1024 KW with KW 1, 3, 16; groups of 256, 512
                                          (300, 1024, 128), (1000, 3072, 256), (77, 16384, 512),
                                          # N <= 8192 and K <= 8192: four T-blocks per wave
                                          # (K 512 KW: 1536, 8192)
                                          (100, 1536, 128), (500, 8192, 128), (8192, 2048, 256),
                                          # K not a multiple of 1024 past N = 8192, or of 512:
                                          # the X-resident kernel at M = 1
                                          (9000, 1536, 128), (250, 1152, 128), (33, 640, 128)])
def test_gemv_shuffled_vs_oracle(gpu, oracle, rows, cols, gs):
    torch = gpu
    packed, scales, zeros = make_int4(rows, cols, gs, seed=rows * 7 + cols)
    xb = normal_bf16((1, cols), seed=cols + 1)
    dp, ds, dz, dx = _dev(torch, packed), _dev(torch, scales), _dev(torch, zeros), _dev_bf16(torch, xb)
    sh = _shuffle(torch, dp, rows, cols)
    y = _host_bf16(_gemm(torch, "kc_gemm_int4_bf16_shuffled", sh, ds, dz, dx, 1, rows, cols, gs))
    truth = oracle.gemm_int4_bf16_f64(packed, scales, zeros.reshape(-1), xb, 1, rows, cols, gs)
    assert rel_l2(y.reshape(1, rows), truth) < 3e-3


@pytest.mark.parametrize("signs", ["ones", "alternating"])
def test_gemv_shuffled_zero_point_identity(gpu, signs):
    """Every nibble equal to its zero point: W = 0.  With x = +-1 every
    matrix-core sum is an exact integer whatever its internal rounding, so
    only the fold's rounding of s (136 + z) remains: |y| <= 1e-6 s 140 sum|x|,
    where a zero point off by one would give s |sum x| (4096 s for ones)."""
    torch = gpu
    rows, cols, gs = 64, 4096, 128
    G = cols // gs
    packed = np.full((rows, cols // 2), 0x33, np.uint8)      # q = 3 everywhere
    zeros = np.full((rows, G // 2), 0x33, np.uint8)          # z = 3 everywhere
    scales = np.full((rows, G), 0.01, np.float32)
    xf = np.ones(cols, np.float32) if signs == "ones" else np.where(np.arange(cols) % 3, 1.0, -1.0).astype(np.float32)
    xb = (xf.view(np.uint32) >> 16).astype(np.uint16).reshape(1, cols)
    dp, ds, dz, dx = _dev(torch, packed), _dev(torch, scales), _dev(torch, zeros), _dev_bf16(torch, xb)
    sh = _shuffle(torch, dp, rows, cols)
    y = _host_bf16(_gemm(torch, "kc_gemm_int4_bf16_shuffled", sh, ds, dz, dx, 1, rows, cols, gs))
    assert np.abs(y).max() <= 1e-6 * 0.01 * 140 * cols


@pytest.mark.parametrize("rows,cols,gs", [(64, 192, 64), (64, 256, 64), (64, 96, 32)])
def test_shuffled_rejects_what_it_cannot_read(gpu, rows, cols, gs):
    """cols not a multiple of 128 (no layout) or groups under 128 (a k-block
    would straddle two scales): KC_ERR_INVALID_ARGUMENT, nothing launched."""
    torch = gpu
    L = _lib()
    buf = torch.zeros(4 * rows * cols, dtype=torch.uint8, device="cuda")
    f = torch.zeros(rows * cols, dtype=torch.float32, device="cuda")
    x = torch.zeros(cols, dtype=torch.bfloat16, device="cuda")
    y = torch.zeros(rows, dtype=torch.bfloat16, device="cuda")
    if cols % 128:
        assert L.kc_shuffled_int4_bytes(rows, cols) == -1
        assert L.kc_shuffle_int4_mfma(ptr(buf), ptr(buf), rows, cols, stream()) == KC_ERR_INVALID_ARGUMENT
        L.kc_get_last_error()
    st = L.kc_gemm_int4_bf16_shuffled(ptr(buf), ptr(f), ptr(buf), ptr(x), ptr(y), 1, rows, cols, gs, stream())
    assert st == KC_ERR_INVALID_ARGUMENT
    assert L.kc_get_last_error() == KC_ERR_INVALID_ARGUMENT
    torch.cuda.synchronize()


def test_shuffle_empty_shapes(gpu):
    torch = gpu
    L = _lib()
    assert L.kc_shuffle_int4_mfma(None, None, 0, 128, stream()) == 0
    assert L.kc_shuffle_int4_mfma(None, None, 16, 0, stream()) == 0
    assert L.kc_shuffled_int4_bytes(0, 128) == 0
    # K = 0: Y = 0 on both layouts, success, no weights read (null pointers)
    for m in (1, 3, 17):
        y0 = torch.full((m, 48), 7.0, dtype=torch.bfloat16, device="cuda")
        y1 = y0.clone()
        assert L.kc_gemm_int4_bf16(None, None, None, None, ptr(y0), m, 48, 0, 128, stream()) == 0
        assert L.kc_gemm_int4_bf16_shuffled(None, None, None, None, ptr(y1), m, 48, 0, 128,
                                            stream()) == 0
        torch.cuda.synchronize()
        assert torch.count_nonzero(y0).item() == 0 and torch.count_nonzero(y1).item() == 0
    torch.cuda.synchronize()
