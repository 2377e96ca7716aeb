"""The reference's Python operators on device tensors: the bridge functions
(kernel_craft_torch_ops, reference src/python/kernel_craft_torch_ops.py:265-381)
and the same ops through torch.ops.kernel_craft dispatch (:428-479), against
the CPU oracle.  Bars: INT4 dequantization, FP8 codes, scales and
dequantization bit for bit; the fp32 GEMV within relative L2 1e-5 of the fp64
oracle.  Re-expressed from the reference's own tests: TestTorchOpsFP8
(test_vllm_backend.py:208-232) and the span emission/attribute cases of
test_otel_e2e.py:192-211,300-331.

Spans: opentelemetry is not importable in this image, so spans are checked
through the tracing module's local records (kernel_craft_otel.recorded_spans):
names, attributes and kernel.cuda_ms.  Export through an OTEL SDK exporter is
not exercised here: parity unpinned for the exporter path.
"""
import numpy as np
import pytest

import kernel_craft_otel as otel
import kernel_craft_torch_ops as ops
from kc_data import make_int4, outlier_activations, rel_l2

pytestmark = pytest.mark.gpu


def _d(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture(params=["bridge", "torch.ops"])
def via(request, gpu):
    """The op table to call: the bridge module or torch.ops.kernel_craft."""
    torch = gpu
    if request.param == "bridge":
        return ops
    assert ops.TORCH_OPS_REGISTERED
    return torch.ops.kernel_craft


@pytest.mark.parametrize("rows,cols,gs", [(256, 512, 128), (96, 4096, 128), (33, 96, 32)])
def test_int4_dequantize_bit_exact(gpu, oracle, via, rows, cols, gs):
    torch = gpu
    p, s, z = make_int4(rows, cols, gs, seed=rows + cols)
    out = via.int4_dequantize(_d(torch, p), _d(torch, s), _d(torch, z), rows, cols, gs)
    assert out.shape == (rows, cols) and out.dtype == torch.float32
    np.testing.assert_array_equal(out.cpu().numpy(),
                                  oracle.dequantize_int4(p, s, z.reshape(-1), rows, cols, gs))


@pytest.mark.parametrize("rows,cols,gs", [(4096, 4096, 128), (256, 512, 128), (100, 1000, 100)])
def test_int4_gemv_vs_oracle(gpu, oracle, via, rows, cols, gs):
    torch = gpu
    p, s, z = make_int4(rows, cols, gs, seed=rows * 3 + cols)
    x = np.random.default_rng(cols).standard_normal(cols).astype(np.float32)
    y = via.int4_gemv(_d(torch, p), _d(torch, s), _d(torch, z), _d(torch, x), rows, cols, gs)
    assert y.shape == (rows,) and y.dtype == torch.float32
    truth = oracle.gemv_int4_f64(p, s, z.reshape(-1), x, rows, cols, gs)
    assert rel_l2(y.cpu().numpy(), truth) < 1e-5


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (8, 64), (5, 1000)])
def test_fp8_quantize_per_token_bit_exact(gpu, oracle, via, rows, cols):
    torch = gpu
    x, _ = outlier_activations(rows, cols, 0.01, 50.0, seed=rows + cols)
    q, s = via.fp8_quantize(_d(torch, x), True)
    assert q.dtype == torch.int8 and q.shape == (rows, cols) and s.shape == (rows,)
    eq, es = oracle.quantize_fp8_per_token(x)
    np.testing.assert_array_equal(s.cpu().numpy(), es)
    np.testing.assert_array_equal(q.cpu().numpy(), eq)


def test_fp8_quantize_per_tensor_saturates(gpu, oracle, via):
    """Per-tensor mode reads its scale from the zeroed scales buffer the op
    allocates (reference :345-347): x / 0 is +-inf or NaN, so every code
    saturates to +-448 (NaN and +0 / 0 -> +448)."""
    torch = gpu
    x = np.random.default_rng(3).standard_normal((16, 128)).astype(np.float32)
    x[0, :4] = [0.0, -0.0, np.nan, np.inf]
    q, s = via.fp8_quantize(_d(torch, x), False)
    assert s.shape == (1,) and s.item() == 0.0
    np.testing.assert_array_equal(q.cpu().numpy(), oracle.quantize_fp8_per_tensor(x, 0.0))


@pytest.mark.parametrize("per_token", [True, False])
def test_fp8_dequantize_bit_exact(gpu, oracle, via, per_token):
    torch = gpu
    rows, cols = 64, 256
    codes = np.random.default_rng(5).integers(-128, 128, (rows, cols), dtype=np.int8)
    codes[codes == 0x7F] = 0          # keep NaN codes out of the fp32 comparison
    codes[codes == -1] = 0
    scales = np.random.default_rng(6).uniform(0.01, 2.0, rows if per_token else 1).astype(np.float32)
    out = via.fp8_dequantize(_d(torch, codes), _d(torch, scales), rows, cols, per_token)
    np.testing.assert_array_equal(out.cpu().numpy(),
                                  oracle.dequantize_fp8(codes, scales, rows, cols, per_token))


class TestTorchOpsFP8:
    """test_vllm_backend.py:208-232 re-expressed (same seeds and bars)."""

    def test_roundtrip_accuracy(self, gpu, via):
        torch = gpu
        x_np = np.random.default_rng(11).uniform(-1, 1, (8, 64)).astype(np.float32)
        q, scales = via.fp8_quantize(torch.tensor(x_np, device="cuda"), True)
        x_hat = via.fp8_dequantize(q, scales, 8, 64, True)
        rel = (x_hat.cpu() - torch.tensor(x_np)).abs() / (torch.tensor(x_np).abs() + 1e-6)
        assert rel.max().item() < 0.15

    def test_output_shapes(self, gpu, via):
        torch = gpu
        x = torch.randn(16, 128, device="cuda")
        q, scales = via.fp8_quantize(x, True)
        assert q.shape == (16, 128) and scales.shape == (16,)
        assert via.fp8_dequantize(q, scales, 16, 128, True).shape == (16, 128)


def test_spans_emitted_with_reference_attributes(gpu):
    """test_otel_e2e.py:192-211 (emission) and :300-331 (attributes): the
    int4_gemv span carries rows, cols, group_size; fp8_quantize carries rows,
    cols, per_token; both get kernel.cuda_ms >= 0 while recorded."""
    torch = gpu
    if otel._HAS_OTEL_API:
        pytest.skip("opentelemetry installed: spans go to the OTEL provider")
    rows, cols, gs = 256, 512, 128
    packed = torch.zeros(rows, cols // 2, dtype=torch.uint8, device="cuda")
    scales = torch.ones(rows, cols // gs, dtype=torch.float32, device="cuda")
    zeros = torch.zeros(rows, cols // gs // 2, dtype=torch.uint8, device="cuda")
    with otel.recorded_spans() as spans:
        ops.int4_gemv(packed, scales, zeros, torch.randn(cols, device="cuda"), rows=rows,
                      cols=cols, group_size=gs)
        ops.fp8_quantize(torch.randn(16, 128, device="cuda"), per_token=True)
    by_name = {s.name: s for s in spans}
    assert set(by_name) == {"int4_gemv", "fp8_quantize"}
    a = by_name["int4_gemv"].attributes
    assert (a["rows"], a["cols"], a["group_size"]) == (rows, cols, gs)
    a = by_name["fp8_quantize"].attributes
    assert (a["rows"], a["cols"], a["per_token"]) == (16, 128, True)
    for span in spans:
        assert span.attributes[otel.CUDA_MS_ATTR] >= 0.0


def test_unrecorded_spans_do_not_synchronize(gpu):
    """Outside a recorder no event is recorded and the host is not blocked:
    a call queued behind a long device sleep returns before it finishes."""
    torch = gpu
    x = torch.randn(8, 64, device="cuda")
    ops.fp8_quantize_rows(x)                      # load the library first
    torch.cuda.synchronize()
    torch.cuda._sleep(200_000_000)                # ~0.1 s of device time
    ops.fp8_quantize_rows(x)
    assert not torch.cuda.current_stream().query(), "the op waited for the device"
    torch.cuda.synchronize()


def test_stub_ops_raise_inside_their_span(gpu):
    """Out-of-scope reference ops: the library's stub reports
    KC_ERR_NOT_IMPLEMENTED, the op raises RuntimeError, and the span the
    reference opens for it is still emitted with its attributes."""
    torch = gpu
    if otel._HAS_OTEL_API:
        pytest.skip("opentelemetry installed")
    Q = torch.randn(1, 4, 32, 64, device="cuda")
    with otel.recorded_spans() as spans:
        with pytest.raises(RuntimeError, match="not implemented|kc_status 2"):
            ops.flash_attention(Q, Q.clone(), Q.clone(), H_kv=4, causal=True)
    assert spans and spans[0].name == "flash_attention"
    assert spans[0].attributes["causal"] is True and spans[0].attributes["head_dim"] == 64


@pytest.mark.parametrize("m,rows,cols", [(4, 300, 2048), (16, 100, 4096), (1, 4096, 4096)])
def test_bridge_shuffled_gemm(gpu, oracle, m, rows, cols):
    """int4_shuffle_mfma + int4_gemm_bf16_shuffled: bit for bit the
    reference-layout int4_gemm_bf16 for m >= 2 at these K (multiples of 1024
    up to 12288: the same K-split kernel reads both layouts); m == 1 (a
    GEMV of its own on each layout) within the bf16 bar of the fp64 oracle."""
    torch = gpu
    gs = 128
    p, s, z = make_int4(rows, cols, gs, seed=rows + m)
    xb = np.random.default_rng(m).standard_normal((m, cols)).astype(np.float32)
    x = torch.from_numpy(xb).cuda().to(torch.bfloat16)
    dp, ds, dz = _d(torch, p), _d(torch, s), _d(torch, z)
    sh = ops.int4_shuffle_mfma(dp, rows, cols)
    assert sh.numel() == (rows + 15) // 16 * 16 * cols // 2
    y = ops.int4_gemm_bf16_shuffled(sh, ds, dz, x, rows, cols, gs)
    if m >= 2:
        assert torch.equal(y.view(torch.int16), ops.int4_gemm_bf16(dp, ds, dz, x, rows, cols, gs).view(torch.int16))
    else:
        xbits = (x.float().cpu().numpy().view(np.uint32) >> 16).astype(np.uint16)
        truth = oracle.gemm_int4_bf16_f64(p, s, z.reshape(-1), xbits, m, rows, cols, gs)
        assert rel_l2(y.float().cpu().numpy().reshape(m, rows), truth) < 3e-3


def test_gemv_chain_non_contiguous_weights(gpu):
    """int4_gemv_bf16_chain with weights that are column slices of wider
    buffers (so the bridge copies them): three ops of one shape and different
    weights, each output bit-identical to int4_gemv_bf16 on contiguous copies
    of the same weights.  The copies must all outlive the library call: with
    same-sized copies freed early, the caching allocator hands op 0's block
    to op 1's copy and op 0 reads op 1's weights."""
    torch = gpu
    from kc_data import normal_bf16
    rows, cols, gs = 1024, 4096, 128
    G = cols // gs
    ops_args, refs = [], []
    for i in range(3):
        p, s, z = make_int4(rows, cols, gs, seed=900 + i)
        wide_p = torch.zeros(rows, cols // 2 + 64, dtype=torch.uint8, device="cuda")
        wide_s = torch.zeros(rows, G + 3, dtype=torch.float32, device="cuda")
        wide_z = torch.zeros(rows, z.shape[1] + 5, dtype=torch.uint8, device="cuda")
        wide_p[:, 32:32 + cols // 2] = _d(torch, p)
        wide_s[:, 1:1 + G] = _d(torch, s)
        wide_z[:, 2:2 + z.shape[1]] = _d(torch, z)
        vp, vs, vz = wide_p[:, 32:32 + cols // 2], wide_s[:, 1:1 + G], wide_z[:, 2:2 + z.shape[1]]
        assert not (vp.is_contiguous() or vs.is_contiguous() or vz.is_contiguous())
        x = _d(torch, normal_bf16((cols,), seed=950 + i).view(np.int16)).view(torch.bfloat16)
        y = torch.empty(rows, dtype=torch.bfloat16, device="cuda")
        ops_args.append((vp, vs, vz, x, y, rows, cols, gs))
        refs.append(ops.int4_gemv_bf16(_d(torch, p), _d(torch, s), _d(torch, z), x, rows, cols, gs))
    ops.int4_gemv_bf16_chain(ops_args)
    torch.cuda.synchronize()
    for i, (args, ref) in enumerate(zip(ops_args, refs)):
        assert torch.equal(args[4].view(torch.int16), ref.view(torch.int16)), f"op {i}"
