"""GPTQ / AWQ checkpoints to the reference INT4 layout.

The source formats are third-party (AutoGPTQ 0.7, AutoAWQ 0.2) and absent
here; the reference has no converter and calls its own layout "GPTQ/AWQ-
style" (quant_int4.cu:5).  The oracle restates their published packing
(oracle/kc_oracle.py: gptq_unpack / awq_unpack); known-answer words pin the
nibble and column order of that restatement, and the converter is pinned by
the dequantization identity: the reference dequantization of the converted
weights (kco_dequantize_int4, quant_int4.cu:79-104) equals (u - zu) * s for
every weight, zero point and scale.  CPU tests check the oracle; GPU tests
compare kc_convert_*_int4 with it bit for bit and run converted weights
through the GEMV."""
import ctypes

import numpy as np
import pytest

from kc_data import bf16_bits_to_f32, normal_bf16, rel_l2


# ---------------------------------------------------------------------------
# CPU: the format restatement and the identity
# ---------------------------------------------------------------------------

def test_gptq_word_order_kat(oracle):
    qweight = np.zeros((1, 8), np.uint32)
    qweight[0, 3] = 0x76543210            # column 3, k = 0..7
    qzeros = np.array([[0xFEDCBA98]], np.uint32)
    u, zu = oracle.gptq_unpack(qweight.view(np.int32), qzeros.view(np.int32), zero_offset=1)
    assert u.shape == (8, 8) and list(u[:, 3]) == list(range(8)) and u[:, [0, 1, 2, 4]].max() == 0
    assert list(zu[0]) == [9, 10, 11, 12, 13, 14, 15, 16]   # stored minus one
    _, zu0 = oracle.gptq_unpack(qweight.view(np.int32), qzeros.view(np.int32), zero_offset=0)
    assert list(zu0[0]) == list(range(8, 16))


def test_awq_column_order_kat(oracle):
    qweight = np.array([[0x76543210]], np.uint32)   # nibble i holds column {0,2,4,6,1,3,5,7}[i]
    u, zu = oracle.awq_unpack(qweight.view(np.int32), qweight.view(np.int32))
    assert list(u[0]) == [0, 4, 1, 5, 2, 6, 3, 7]
    assert list(zu[0]) == [0, 4, 1, 5, 2, 6, 3, 7]


@pytest.mark.parametrize("fmt", ["gptq1", "gptq2", "awq"])
def test_pack_unpack_round_trip(oracle, fmt):
    rng = np.random.default_rng(3)
    K, N, G = 256, 48, 4
    u = rng.integers(0, 16, (K, N)).astype(np.uint8)
    if fmt == "awq":
        zu = rng.integers(0, 16, (G, N)).astype(np.int32)
        u2, z2 = oracle.awq_unpack(*oracle.awq_pack(u, zu))
    else:
        off = 1 if fmt == "gptq1" else 0
        zu = rng.integers(off, 16 + off, (G, N)).astype(np.int32)
        u2, z2 = oracle.gptq_unpack(*oracle.gptq_pack(u, zu, off), zero_offset=off)
    np.testing.assert_array_equal(u2, u)
    np.testing.assert_array_equal(z2, zu)


def _case(rng, K, N, gs, zlo, zhi):
    G = K // gs
    u = rng.integers(0, 16, (K, N)).astype(np.uint8)
    zu = rng.integers(zlo, zhi + 1, (G, N)).astype(np.int32)
    if N >= zhi - zlo + 1:
        zu[:, :zhi - zlo + 1] = np.arange(zlo, zhi + 1)   # every zero point occurs
    s16 = rng.uniform(0.001, 0.05, (G, N)).astype(np.float16)
    s16[0, :4] = np.array([1.0, -0.5, 6e-8, 65504.0], np.float16)  # sign, subnormal, max
    return u, zu, s16


@pytest.mark.parametrize("zlo,zhi", [(0, 15), (1, 16)])
def test_convert_identity_every_zero_point(oracle, zlo, zhi):
    rng = np.random.default_rng(zlo + 10)
    K, N, gs = 512, 64, 128
    u, zu, s16 = _case(rng, K, N, gs, zlo, zhi)
    W = oracle.int4_source_dequant(u, zu, s16, group_size=gs).T
    p, s, z = oracle.convert_to_reference(u, zu, s16, group_size=gs)
    Wr = oracle.dequantize_int4(p, s, z.reshape(-1), N, K, gs)
    np.testing.assert_array_equal(Wr, W)            # equal as numbers
    # bits differ only in the sign of a zero (a negated scale flips it)
    diff = Wr.view(np.uint32) != W.view(np.uint32)
    assert np.all(W[diff] == 0) and np.all(Wr[diff] == 0)
    assert np.all(np.signbit(Wr[diff]) != np.signbit(W[diff]))


def test_convert_act_order_permutation(oracle):
    rng = np.random.default_rng(21)
    K, N, gs = 512, 32, 128
    G = K // gs
    g_idx = np.repeat(np.arange(G), gs)
    rng.shuffle(g_idx)                               # act-order: groups scattered over k
    u = rng.integers(0, 16, (K, N)).astype(np.uint8)
    zu = rng.integers(1, 17, (G, N)).astype(np.int32)
    s16 = rng.uniform(0.001, 0.05, (G, N)).astype(np.float16)
    perm = np.argsort(g_idx, kind="stable")
    W = oracle.int4_source_dequant(u, zu, s16, g_idx=g_idx, group_size=gs)   # [K, N]
    p, s, z = oracle.convert_to_reference(u, zu, s16, perm=perm, group_size=gs)
    Wr = oracle.dequantize_int4(p, s, z.reshape(-1), N, K, gs)               # [N, K]
    np.testing.assert_array_equal(Wr, W[perm].T)
    x = rng.standard_normal(K)
    np.testing.assert_allclose(Wr.astype(np.float64) @ x[perm], W.T.astype(np.float64) @ x, rtol=1e-12)


def test_act_order_permutation_helper():
    torch = pytest.importorskip("torch")
    import kernel_craft_torch_ops as ops
    K, gs = 512, 128
    assert ops.act_order_permutation(torch.arange(K) // gs, gs) is None
    g = torch.arange(K) // gs
    g = g[torch.randperm(K, generator=torch.Generator().manual_seed(0))]
    perm = ops.act_order_permutation(g, gs)
    assert perm.dtype == torch.int32
    assert torch.equal(g[perm.long()], torch.arange(K) // gs)
    bad = g.clone()
    bad[0] = (bad[0] + 1) % (K // gs)
    with pytest.raises(ValueError):
        ops.act_order_permutation(bad, gs)


# ---------------------------------------------------------------------------
# GPU: kc_convert_gptq_int4 / kc_convert_awq_int4 against the oracle
# ---------------------------------------------------------------------------

def _to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    return t.cpu().numpy()


SHAPES = [(256, 64, 128), (4096, 4096, 128), (1024, 136, 32), (512, 72, 64), (896, 24, 64),
          (4096, 448, 256),
          (208, 136, 8)]  # K/8 = 26 words: the word-by-word stores; a partial 128-column tile


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,gs", SHAPES)
@pytest.mark.parametrize("fmt", ["gptq1", "gptq2", "awq"])
def test_gpu_convert_matches_oracle(gpu, oracle, K, N, gs, fmt):
    torch = gpu
    import kernel_craft_torch_ops as ops
    rng = np.random.default_rng(K + N + gs)
    off = {"gptq1": 1, "gptq2": 0, "awq": 0}[fmt]
    u, zu, s16 = _case(rng, K, N, gs, off, 15 + off)
    print(f"convert {fmt} K={K} N={N} gs={gs}", flush=True)
    if fmt == "awq":
        qw, qz = oracle.awq_pack(u, zu)
        p, s, z = ops.convert_awq(_to_dev(torch, qw), _to_dev(torch, qz),
                                  _to_dev(torch, s16.view(np.int16)).view(torch.float16), gs)
    else:
        qw, qz = oracle.gptq_pack(u, zu, off)
        p, s, z, perm = ops.convert_gptq(_to_dev(torch, qw), _to_dev(torch, qz),
                                         _to_dev(torch, s16.view(np.int16)).view(torch.float16),
                                         None, gs, off)
        assert perm is None
    torch.cuda.synchronize()
    ep, es, ez = oracle.convert_to_reference(u, zu, s16, group_size=gs)
    np.testing.assert_array_equal(_host(p), ep)
    np.testing.assert_array_equal(_host(s).view(np.uint32), es.view(np.uint32))
    np.testing.assert_array_equal(_host(z), ez)


@pytest.mark.gpu
def test_gpu_convert_act_order_then_gemv(gpu, oracle):
    torch = gpu
    import kernel_craft_torch_ops as ops
    rng = np.random.default_rng(9)
    K, N, gs = 2048, 512, 128
    G = K // gs
    g_idx = np.repeat(np.arange(G), gs)
    rng.shuffle(g_idx)
    u = rng.integers(0, 16, (K, N)).astype(np.uint8)
    zu = rng.integers(1, 17, (G, N)).astype(np.int32)
    s16 = rng.uniform(0.001, 0.05, (G, N)).astype(np.float16)
    qw, qz = oracle.gptq_pack(u, zu, 1)
    print("convert gptq act-order then GEMV", flush=True)
    p, s, z, perm = ops.convert_gptq(_to_dev(torch, qw), _to_dev(torch, qz),
                                     _to_dev(torch, s16.view(np.int16)).view(torch.float16),
                                     torch.from_numpy(g_idx.astype(np.int32)), gs, 1)
    assert perm is not None
    hperm = _host(perm)
    np.testing.assert_array_equal(hperm, np.argsort(g_idx, kind="stable"))
    ep, es, ez = oracle.convert_to_reference(u, zu, s16, perm=hperm, group_size=gs)
    np.testing.assert_array_equal(_host(p), ep)
    np.testing.assert_array_equal(_host(s).view(np.uint32), es.view(np.uint32))
    np.testing.assert_array_equal(_host(z), ez)
    # the converted layer through the bf16 GEMV, x permuted as the layout asks
    xb = normal_bf16(K, seed=4)
    x = bf16_bits_to_f32(xb)
    y = ops.int4_gemv_bf16(p, s, z, _to_dev(torch, xb.view(np.int16)).view(torch.bfloat16)[perm.long()],
                           N, K, gs)
    truth = oracle.int4_source_dequant(u, zu, s16, g_idx=g_idx, group_size=gs).astype(np.float64).T @ x
    yf = y.float().cpu().numpy()
    assert rel_l2(yf, truth) < 3e-3


@pytest.mark.gpu
def test_gpu_convert_argument_errors(gpu):
    import kc_abi
    L = kc_abi.lib()
    cases = [(1024, 64, 512, 1),   # K / gs = 2 groups: fine -> then odd groups below
             (1536, 64, 512, 1),   # 3 groups: odd
             (1020, 64, 128, 1),   # K % 8
             (1024, 60, 128, 1),   # N % 8
             (1024, 64, 100, 1),   # gs % 8
             (1024, 64, 128, 2)]   # zero_offset
    dummy = ctypes.c_void_p(16)
    for i, (K, N, gs, off) in enumerate(cases[1:]):
        st = L.kc_convert_gptq_int4(dummy, dummy, dummy, None, K, N, gs, off, dummy, dummy, dummy,
                                    None)
        assert st == 1, (K, N, gs, off)
        L.kc_get_last_error()
    st = L.kc_convert_awq_int4(None, dummy, dummy, 1024, 64, 128, dummy, dummy, dummy, None)
    assert st == 1
    L.kc_get_last_error()
