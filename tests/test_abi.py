"""C ABI and host-bridge checks that need no GPU.

The library is loaded exactly as the reference's ctypes bridge loads it
(kernel_craft_torch_ops.py:93-98).  Only calls that return before any HIP
call are made here: stubs and argument validation.
"""
import ctypes
import importlib
import os
import subprocess
import sys

import pytest
import torch

import kc_abi
import kernel_craft_torch_ops as ops

# The symbols the reference's loaders bind (kernel_craft_torch_ops.py:101-168
# and pybind_transformer.cpp:36-122); a drop-in library must export them all.
REFERENCE_BRIDGE_SYMBOLS = [
    "launch_flash_attention", "launch_paged_attention", "launch_dequantize_int4",
    "launch_gemv_int4", "launch_quantize_fp8", "launch_dequantize_fp8",
    "launch_verify_draft_tokens",
]
REFERENCE_PYBIND_SYMBOLS = REFERENCE_BRIDGE_SYMBOLS + [
    "launch_smoothquant_scale", "launch_compute_prefix_length", "launch_ring_allreduce",
    "launch_allgather", "launch_col_parallel_linear", "launch_row_parallel_linear",
    "launch_selective_scan", "launch_depthwise_conv1d", "launch_rmsnorm",
    "nccl_comm_init_all", "nccl_comm_destroy", "nccl_group_start", "nccl_group_end",
    "launch_ring_allreduce_nccl", "launch_allgather_nccl", "nccl_comm_count",
    "nccl_comm_user_rank",
]


@pytest.fixture(scope="module")
def lib():
    return kc_abi.lib()


def test_library_exports_every_header_symbol(lib):
    declared = kc_abi.header_functions()
    assert len(declared) >= 35
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing


def test_reference_loaders_find_their_symbols(lib):
    for name in REFERENCE_PYBIND_SYMBOLS:
        assert hasattr(lib, name), name


def test_exported_set_equals_header():
    out = subprocess.run(["nm", "-D", "--defined-only", str(kc_abi.ROOT / "build" / "libkernels.so")],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines()
                if line.split()[-1].startswith(("launch_", "kc_", "nccl_"))}
    assert exported == set(kc_abi.header_functions())


def test_stubs_report_not_implemented(lib, capfd):
    lib.kc_get_last_error()
    lib.launch_flash_attention(None, None, None, None, 1, 1, 1, 1, 1, False, None)
    assert "[kernel-craft-hip stub] launch_flash_attention not implemented" in capfd.readouterr().err
    assert lib.kc_peek_last_error() == 2
    assert b"launch_flash_attention" in lib.kc_last_error_string()
    assert lib.kc_get_last_error() == 2
    assert lib.kc_get_last_error() == 0
    lib.launch_depthwise_conv1d.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 4 + [
        ctypes.c_void_p]
    lib.launch_depthwise_conv1d(None, None, None, None, 1, 1, 1, 1, None)
    assert lib.kc_get_last_error() == 2
    lib.nccl_comm_count.restype = ctypes.c_int
    lib.nccl_comm_user_rank.restype = ctypes.c_int
    assert lib.nccl_comm_count(None) == 0 and lib.nccl_comm_user_rank(None) == -1


@pytest.mark.parametrize("rows,cols,gs,why", [
    (4, 7, 1, "even"),            # odd cols
    (4, 256, 96, "divide"),       # group size does not divide cols
    (4, 256, 0, "> 0"),
    (-1, 256, 128, "negative"),
])
def test_int4_argument_validation(lib, rows, cols, gs, why):
    lib.kc_get_last_error()
    p = ctypes.c_void_p(0x1000)   # never dereferenced: validation fails first
    lib.launch_gemv_int4(p, p, p, p, p, rows, cols, gs, None)
    assert lib.kc_peek_last_error() == 1
    assert why in lib.kc_last_error_string().decode()
    lib.kc_get_last_error()
    lib.launch_dequantize_int4(p, p, p, p, rows, cols, gs, None)
    assert lib.kc_get_last_error() == 1
    assert lib.kc_gemv_int4_bf16(p, p, p, p, p, rows, cols, gs, None) == 1
    lib.kc_get_last_error()


def test_null_pointers_rejected(lib):
    lib.kc_get_last_error()
    lib.launch_gemv_int4(None, None, None, None, None, 4, 256, 128, None)
    assert lib.kc_get_last_error() == 1
    lib.launch_quantize_fp8(None, None, None, 4, 64, True, None)
    assert lib.kc_get_last_error() == 1
    assert lib.kc_quantize_fp8_smooth_div_bf16(None, None, None, None, 4, 64, None) == 1
    assert lib.kc_gemm_int4_bf16(None, None, None, None, None, 65, 4, 256, 128, None) == 1
    lib.kc_get_last_error()


def test_empty_shapes_are_noops(lib):
    """rows == 0 (and FP8 cols == 0) launch nothing and report success.  The
    reference-named launchers still synchronize their stream (a HIP call), so
    they are checked in the GPU suite; the stream-ordered entry points return
    before any HIP call."""
    lib.kc_get_last_error()
    assert lib.kc_gemv_int4_bf16(None, None, None, None, None, 0, 256, 128, None) == 0
    assert lib.kc_gemv_int4_f32_async(None, None, None, None, None, 0, 256, 128, None) == 0
    assert lib.kc_gemm_int4_bf16(None, None, None, None, None, 0, 64, 256, 128, None) == 0
    assert lib.kc_quantize_fp8_per_token_f32(None, None, None, 0, 64, None) == 0
    assert lib.kc_quantize_fp8_per_token_bf16(None, None, None, 5, 0, None) == 0
    assert lib.kc_quantize_fp8_smooth_mul_bf16(None, None, None, None, 0, 64, None) == 0
    assert lib.kc_get_last_error() == 0


def test_bridge_prototypes_and_discovery(tmp_path, monkeypatch):
    ops._setup_prototypes(kc_abi.lib())
    for name in REFERENCE_BRIDGE_SYMBOLS:
        assert name in ops.PROTOTYPES
    # KERNEL_CRAFT_LIB wins when it exists (reference :71-72)
    fake = tmp_path / "libkernels.so"
    fake.write_bytes(b"")
    monkeypatch.setenv("KERNEL_CRAFT_LIB", str(fake))
    assert ops._find_lib() == str(fake)
    monkeypatch.setenv("KERNEL_CRAFT_LIB", str(tmp_path / "absent.so"))
    assert ops._find_lib().endswith(os.path.join("build", "libkernels.so"))


def test_bridge_fails_loudly_without_library(tmp_path):
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "import kernel_craft_torch_ops as o\n"
        "o._find_lib = lambda: (_ for _ in ()).throw(FileNotFoundError('libkernels.so not found'))\n"
        "import torch\n"
        "try:\n"
        "    o._get_lib()\n"
        "except FileNotFoundError as e:\n"
        "    print('raised', e)\n" % str(kc_abi.ROOT / "kernel-craft_amd" / "python"))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True)
    assert "raised libkernels.so not found" in out.stdout


def test_torch_library_schemas():
    assert ops.TORCH_OPS_REGISTERED
    for name, schema in ops.SCHEMAS.items():
        op = getattr(torch.ops.kernel_craft, name)
        assert str(op.default._schema) == "kernel_craft::" + schema


def test_cpu_tensors_rejected():
    x = torch.zeros(4, 64)
    with pytest.raises(ValueError, match="GPU only"):
        ops.fp8_quantize(x)
    with pytest.raises(ValueError, match="GPU only"):
        torch.ops.kernel_craft.fp8_quantize(x, True)


def test_otel_local_spans_record_only_inside_a_recorder():
    """Without opentelemetry-api, spans are local records: attributes (and
    device timing) only while a recorded_spans() block collects them."""
    import kernel_craft_otel as otel
    importlib.reload(otel)
    if otel._HAS_OTEL_API:
        pytest.skip("opentelemetry-api is installed: spans come from OTEL")
    with otel.kernel_span("int4_gemv", rows=256, cols=512, group_size=128) as span:
        pass
    assert not span.is_recording() and span.attributes == {}
    with otel.recorded_spans() as spans:
        with otel.kernel_span("int4_gemv", rows=256, cols=512, group_size=128):
            with otel.kernel_span("fp8_quantize", rows=16, cols=128, per_token=True):
                pass
    assert [s.name for s in spans] == ["fp8_quantize", "int4_gemv"]
    assert spans[1].attributes == {"rows": 256, "cols": 512, "group_size": 128}
    assert spans[0].attributes["per_token"] is True
    # no GPU here: no device timing, so no kernel.cuda_ms
    assert otel.CUDA_MS_ATTR not in spans[0].attributes
    assert spans[0].end_ns >= spans[0].start_ns
    otel.setup_tracing()   # no-op without opentelemetry; must not raise


def test_otel_timer_skips_capture_and_missing_gpu(monkeypatch):
    """Device timing is never attempted while the stream is being captured
    into a graph, nor without a visible GPU."""
    import kernel_craft_otel as otel
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    assert otel._DeviceTimer.begin() is None
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    assert otel._DeviceTimer.begin() is None


def test_bridge_span_fallback_accepts_attributes(tmp_path):
    """If the tracing module cannot be imported, the bridge's stand-in span
    takes the same keyword attributes and does nothing."""
    code = (
        "import sys, builtins; sys.path.insert(0, %r)\n"
        "real = builtins.__import__\n"
        "def imp(name, *a, **k):\n"
        "    if name == 'kernel_craft_otel': raise ImportError(name)\n"
        "    return real(name, *a, **k)\n"
        "builtins.__import__ = imp\n"
        "import kernel_craft_torch_ops as o\n"
        "with o.kernel_span('int4_gemv', rows=1, cols=2, group_size=3) as s:\n"
        "    print('ok', s)\n" % str(kc_abi.ROOT / "kernel-craft_amd" / "python"))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True)
    assert "ok None" in out.stdout, out.stderr


@pytest.mark.parametrize("call, match", [
    (lambda: ops.int4_gemv(torch.zeros(8, 64, dtype=torch.uint8), torch.zeros(8, 1),
                           torch.zeros(8, 1, dtype=torch.uint8),
                           torch.zeros(128, dtype=torch.float16), 8, 128, 128), "dtype"),
    (lambda: ops.int4_gemv(torch.zeros(8, 64, dtype=torch.uint8), torch.zeros(8, 1),
                           torch.zeros(8, 1, dtype=torch.uint8), torch.zeros(64), 8, 128, 128),
     "elements"),
    # one group per row: the zero row stride is 0 and every row reads byte 0
    (lambda: ops.int4_gemv(torch.zeros(8, 64, dtype=torch.uint8), torch.zeros(8, 1),
                           torch.zeros(8, 0, dtype=torch.uint8), torch.zeros(128), 8, 128, 128),
     "zeros"),
    # three groups: stride 1, the last row reads byte 7 + 1
    (lambda: ops.int4_gemv(torch.zeros(8, 192, dtype=torch.uint8), torch.zeros(8, 3),
                           torch.zeros(8, dtype=torch.uint8), torch.zeros(384), 8, 384, 128),
     "zeros"),
    (lambda: ops.int4_gemv_bf16(torch.zeros(8, 64, dtype=torch.uint8), torch.zeros(8, 1),
                                torch.zeros(8, 1, dtype=torch.uint8), torch.zeros(128),
                                8, 128, 128), "dtype"),
    (lambda: ops.int4_gemv_bf16(torch.zeros(8, 32, dtype=torch.uint8), torch.zeros(8, 1),
                                torch.zeros(8, 1, dtype=torch.uint8),
                                torch.zeros(128, dtype=torch.bfloat16), 8, 128, 128), "elements"),
    (lambda: ops.int4_gemm_bf16(torch.zeros(8, 64, dtype=torch.uint8), torch.zeros(8, 1),
                                torch.zeros(8, 1, dtype=torch.uint8),
                                torch.zeros(4, 128, dtype=torch.bfloat16), 8, 128, 64), "scales"),
    (lambda: ops.rmsnorm_int4_gemv_bf16(torch.zeros(128, dtype=torch.float16),
                                        torch.zeros(128, dtype=torch.bfloat16),
                                        torch.zeros(8, 64, dtype=torch.uint8), torch.zeros(8, 1),
                                        torch.zeros(8, 1, dtype=torch.uint8), 8, 128, 128),
     "dtype"),
    (lambda: ops.fp8_quantize_rows(torch.zeros(4, 64, dtype=torch.float16)), "dtype"),
    (lambda: ops.col_absmax(torch.zeros(4, 64, dtype=torch.float16)), "dtype"),
    (lambda: ops.fp8_quantize_smooth(torch.zeros(4, 64, dtype=torch.float16), torch.ones(64)),
     "dtype"),
    (lambda: ops.fp8_quantize_smooth(torch.zeros(4, 64), torch.ones(64), mode="mul"), "dtype"),
    (lambda: ops.fp8_quantize_smooth(torch.zeros(4, 64, dtype=torch.bfloat16), torch.ones(32)),
     "elements"),
    (lambda: ops.fp8_quantize(torch.zeros(4, 64, dtype=torch.bfloat16)), "dtype"),
    (lambda: ops.fp8_dequantize(torch.zeros(4, 64, dtype=torch.int8), torch.ones(3), 4, 64),
     "elements"),
    (lambda: ops.fp8_gemm_w8a8(torch.zeros(4, 64, dtype=torch.int8), torch.ones(4),
                               torch.zeros(8, 32, dtype=torch.int8), torch.ones(8)), "share K"),
    (lambda: ops.smooth_factors(torch.ones(8), torch.ones(7)), "elements"),
    (lambda: ops.smoothquant_stats(torch.zeros(4, 64, dtype=torch.float16),
                                   torch.zeros(8, 64, dtype=torch.float16)), "dtype"),
    (lambda: ops.smoothquant_stats(torch.zeros(4, 64, dtype=torch.bfloat16), torch.zeros(8, 64)),
     "dtype"),
    (lambda: ops.smoothquant_stats(torch.zeros(4, 64), torch.zeros(8, 32)), "same number of columns"),
    (lambda: ops.smoothquant_stats(torch.zeros(4, 64), torch.zeros(8, 64)), "GPU only"),
    (lambda: ops.rmsnorm(torch.zeros(2, 64, dtype=torch.float16), torch.ones(64)), "dtype"),
    (lambda: ops.int4_shuffle_mfma(torch.zeros(8, 48, dtype=torch.uint8), 8, 96), "multiple of 128"),
    (lambda: ops.int4_shuffle_mfma(torch.zeros(8, 32, dtype=torch.uint8), 8, 128), "elements"),
    (lambda: ops.int4_gemm_bf16_shuffled(torch.zeros(8 * 64, dtype=torch.uint8), torch.zeros(8, 1),
                                         torch.zeros(8, 1, dtype=torch.uint8),
                                         torch.zeros(4, 128, dtype=torch.bfloat16), 9, 128, 128),
     "elements"),
    (lambda: ops.int4_gemm_bf16_shuffled(torch.zeros(16 * 64, dtype=torch.uint8), torch.zeros(16, 1),
                                         torch.zeros(16, 1, dtype=torch.uint8),
                                         torch.zeros(4, 128, dtype=torch.float16), 16, 128, 128),
     "dtype"),
])
def test_bridge_validates_inputs_before_launch(call, match):
    """Wrong dtypes and sizes are rejected on the host with ValueError before
    any pointer reaches a kernel (a bf16 read of an fp16 buffer is fine, an
    fp32 read of it runs past its end)."""
    with pytest.raises(ValueError, match=match):
        call()
