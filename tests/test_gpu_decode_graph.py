"""A Llama-3-8B decode layer's quantized linears captured in a HIP graph.

The layer is the four INT4 projections at their decode shapes (group 128),
wired as in a decoder with the parts outside this path stood in by slices:

    qkv  = W_qkv  x1,   x1 = bf16(gamma1 * h)  scaled by rms_inv(h)   (fused RMSNorm-GEMV)
    o    = W_o    qkv[:4096]                    (attention output stand-in)
    gu   = W_gu   x2,   x2 = bf16(gamma2 * o)  scaled by rms_inv(o)   (fused RMSNorm-GEMV)
    down = W_down gu[:14336]                    (activation output stand-in)

Captured with torch.cuda.graph on a side stream and replayed several times,
with eager work on the same buffers between replays (outputs overwritten,
the input changed).  Every replay must equal the eager launches bit for bit,
and each stage must lie within relative L2 3e-3 of the fp64 oracle of its own
bf16 input.  The same for kc_gemv_int4_bf16_chain (the four GEMVs from one
call, each taking the previous one's output) and for the FP8 prologue
(kc_rmsnorm_quantize_fp8_bf16 feeding kc_gemm_fp8_w8a8_bf16).
"""
import ctypes

import numpy as np
import pytest

import kc_abi
import kernel_craft_torch_ops as ops
from kc_abi import ptr
from kc_data import bf16_bits_to_f32, f32_to_bf16_bits, make_int4, normal_bf16, rel_l2

pytestmark = pytest.mark.gpu

GS = 128
SHAPES = {"qkv": (6144, 4096), "o": (4096, 4096), "gu": (28672, 4096), "down": (4096, 14336)}


def _bits(t):
    import torch
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _dev_bf16(torch, bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


@pytest.fixture(scope="module")
def layer(gpu):
    torch = gpu
    host, dev = {}, {}
    for i, (name, (n, k)) in enumerate(SHAPES.items()):
        p, s, z = make_int4(n, k, GS, seed=300 + i)
        host[name] = (p, s, z)
        dev[name] = tuple(torch.from_numpy(a).cuda() for a in (p, s, z))
    rng = np.random.default_rng(310)
    g1 = f32_to_bf16_bits(rng.uniform(0.5, 1.5, 4096).astype(np.float32))
    g2 = f32_to_bf16_bits(rng.uniform(0.5, 1.5, 4096).astype(np.float32))
    return host, dev, g1, g2


def _stage_truth(oracle, host, name, x_bits, gamma_bits=None, eps=1e-5):
    """fp64 oracle of one stage from its own bf16 input (and, fused, the
    RMSNorm scale applied to the row sums of W bf16(gamma x))."""
    n, k = SHAPES[name]
    p, s, z = host[name]
    x = bf16_bits_to_f32(x_bits)
    if gamma_bits is None:
        return oracle.gemv_int4_f64(p, s, z.reshape(-1), x, n, k, GS)
    rinv = 1.0 / np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps)
    xg = bf16_bits_to_f32(f32_to_bf16_bits(bf16_bits_to_f32(gamma_bits) * x))
    return oracle.gemv_int4_f64(p, s, z.reshape(-1), xg, n, k, GS) * rinv


def test_decode_layer_graph_replays_match_eager(gpu, oracle, layer):
    torch = gpu
    host, dev, g1b, g2b = layer
    L = kc_abi.lib()
    h = _dev_bf16(torch, normal_bf16((4096,), seed=311))
    g1, g2 = _dev_bf16(torch, g1b), _dev_bf16(torch, g2b)
    out = {name: torch.empty(n, dtype=torch.bfloat16, device="cuda")
           for name, (n, _) in SHAPES.items()}
    eps = 1e-5

    def layer_step():
        s = torch.cuda.current_stream().cuda_stream
        sts = [
            L.kc_rmsnorm_gemv_int4_bf16(ptr(h), ptr(g1), eps, *map(ptr, dev["qkv"]),
                                        ptr(out["qkv"]), 6144, 4096, GS, s),
            L.kc_gemv_int4_bf16(*map(ptr, dev["o"]), ptr(out["qkv"]), ptr(out["o"]),
                                4096, 4096, GS, s),
            L.kc_rmsnorm_gemv_int4_bf16(ptr(out["o"]), ptr(g2), eps, *map(ptr, dev["gu"]),
                                        ptr(out["gu"]), 28672, 4096, GS, s),
            L.kc_gemv_int4_bf16(*map(ptr, dev["down"]), ptr(out["gu"]), ptr(out["down"]),
                                4096, 14336, GS, s),
        ]
        assert not any(sts), L.kc_last_error_string()

    def check_against_oracle(res, h_bits):
        stages = [("qkv", h_bits, g1b), ("o", res["qkv"][:4096], None),
                  ("gu", res["o"], g2b), ("down", res["gu"][:14336], None)]
        for name, xin, gam in stages:
            truth = _stage_truth(oracle, host, name, xin, gam, eps)
            err = rel_l2(bf16_bits_to_f32(res[name]), truth)
            assert err < 3e-3, (name, err)

    print("decode layer: eager", flush=True)
    layer_step()
    torch.cuda.synchronize()
    eager = {k: _bits(v) for k, v in out.items()}
    check_against_oracle(eager, _bits(h))

    print("decode layer: capture", flush=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            layer_step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    for rep in range(3):
        print(f"decode layer: replay {rep}", flush=True)
        for v in out.values():
            v.fill_(float("nan"))          # eager work on the replay's buffers
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k, v in out.items():
            np.testing.assert_array_equal(_bits(v), eager[k], err_msg=f"replay {rep} {k}")

    # a new input: the replay reads the buffer, not a captured copy
    print("decode layer: replay with a new input", flush=True)
    h.copy_(_dev_bf16(torch, normal_bf16((4096,), seed=312)))
    graph.replay()
    torch.cuda.synchronize()
    replayed = {k: _bits(v) for k, v in out.items()}
    layer_step()
    torch.cuda.synchronize()
    for k, v in out.items():
        np.testing.assert_array_equal(replayed[k], _bits(v), err_msg=k)
    assert not np.array_equal(replayed["qkv"], eager["qkv"])
    check_against_oracle(replayed, _bits(h))


def test_gemv_chain_graph_replays_match_eager(gpu, oracle, layer):
    """kc_gemv_int4_bf16_chain under capture: the four GEMVs, each op's x a
    slice of the previous op's y, replayed bit-identical to the eager call."""
    torch = gpu
    host, dev, _, _ = layer
    x0 = _dev_bf16(torch, normal_bf16((4096,), seed=313))
    out = {name: torch.empty(n, dtype=torch.bfloat16, device="cuda")
           for name, (n, _) in SHAPES.items()}
    xin = {"qkv": x0, "o": out["qkv"][:4096], "gu": out["o"], "down": out["gu"][:14336]}
    chain = [(*dev[name], xin[name], out[name], n, k, GS) for name, (n, k) in SHAPES.items()]

    print("gemv chain: eager", flush=True)
    ops.int4_gemv_bf16_chain(chain)
    torch.cuda.synchronize()
    eager = {k: _bits(v) for k, v in out.items()}
    for name in SHAPES:
        x_bits = _bits(x0) if name == "qkv" else _bits(xin[name])
        truth = _stage_truth(oracle, host, name, x_bits)
        assert rel_l2(bf16_bits_to_f32(eager[name]), truth) < 3e-3, name

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    print("gemv chain: capture", flush=True)
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            ops.int4_gemv_bf16_chain(chain)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"gemv chain: replay {rep}", flush=True)
        for v in out.values():
            v.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k, v in out.items():
            np.testing.assert_array_equal(_bits(v), eager[k], err_msg=f"replay {rep} {k}")


def test_fp8_prologue_and_gemm_graph(gpu, oracle):
    """RMSNorm -> FP8 per-token codes -> W8A8 GEMM, captured and replayed:
    bit-identical to eager, codes bit-exact against the oracle composition."""
    torch = gpu
    T, D, N = 64, 4096, 1024
    hb = normal_bf16((T, D), seed=320)
    gb = f32_to_bf16_bits(np.random.default_rng(321).uniform(0.5, 1.5, D).astype(np.float32))
    h, g = _dev_bf16(torch, hb), _dev_bf16(torch, gb)
    w = _dev_bf16(torch, normal_bf16((N, D), seed=322, std=0.02))
    qw, sw = ops.fp8_quantize_rows(w)
    qx = torch.empty(T, D, dtype=torch.int8, device="cuda")
    sx = torch.empty(T, dtype=torch.float32, device="cuda")
    y = torch.empty(T, N, dtype=torch.bfloat16, device="cuda")
    L = kc_abi.lib()

    def step():
        s = torch.cuda.current_stream().cuda_stream
        assert L.kc_rmsnorm_quantize_fp8_bf16(ptr(h), ptr(g), 1e-6, ptr(qx), ptr(sx), T, D, s) == 0
        assert L.kc_gemm_fp8_w8a8_bf16(ptr(qx), ptr(sx), ptr(qw), ptr(sw), ptr(y), T, N, D, s) == 0

    print("fp8 prologue + gemm: eager", flush=True)
    step()
    torch.cuda.synchronize()
    eq, es = oracle.rmsnorm_quantize_fp8_bf16(hb, gb, 1e-6)
    np.testing.assert_array_equal(qx.cpu().numpy(), eq)
    np.testing.assert_array_equal(sx.cpu().numpy(), es)
    y_eager = _bits(y)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    print("fp8 prologue + gemm: capture", flush=True)
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"fp8 prologue + gemm: replay {rep}", flush=True)
        qx.zero_()
        y.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(qx.cpu().numpy(), eq)
        np.testing.assert_array_equal(_bits(y), y_eager)
