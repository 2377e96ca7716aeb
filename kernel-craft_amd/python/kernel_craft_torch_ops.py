"""
kernel_craft_torch_ops.py
PyTorch operators over libkernels.so, the MI355X (gfx950) HIP build of
kernel-craft's quantized-inference kernels, loaded through ctypes.

The module keeps the interface of kernel-craft's bridge
(``src/python/kernel_craft_torch_ops.py``):

* the library is found through ``KERNEL_CRAFT_LIB``, then
  ``../../build/libkernels.so``, ``../../libkernels.so`` and
  ``/usr/local/lib/kernel_craft/libkernels.so`` relative to this file
  (reference :68-87), and loaded with ``RTLD_GLOBAL`` (:96);
* the seven symbols the reference binds on load (:101-168) are bound here
  too, so a library missing any of them fails every op, as there;
* the public operators keep their names, arguments, output allocations and
  span names/attributes (:193-421);
* ``torch.ops.kernel_craft.*`` is registered with the reference's schema
  strings for the CPU and CUDA dispatch keys (:428-479).

On ROCm PyTorch a GPU tensor has ``device.type == "cuda"`` and
``torch.cuda.current_stream().cuda_stream`` is a ``hipStream_t``.

What this module adds:

* every input is checked (device, dtype, element count against the shape
  arguments) before anything is launched, and a mismatch raises
  ``ValueError``: the kernels trust the pointers they are given;
* the library's error channel (``kc_get_last_error``) is read after each
  call and a failure raises ``RuntimeError``;
* there is no CPU fallback: a CPU tensor is an error;
* operators for the entry points the reference lacks (bf16 GEMV and its
  chain, the M > 1 GEMM, RMSNorm and its fusions, bf16 and fused-SmoothQuant
  FP8 quantization, the FP8 GEMM, checkpoint conversion).

Usage
-----
::

    import kernel_craft_torch_ops as kc_ops
    y = kc_ops.int4_gemv(packed, scales, zeros, x, rows, cols, group_size=128)
    q, scales = kc_ops.fp8_quantize(x, per_token=True)
    x_hat     = kc_ops.fp8_dequantize(q, scales, rows, cols, per_token=True)

Build the library with ``make -C kernel-craft_amd`` (writes
``build/libkernels.so``).
"""

import contextlib
import ctypes
import os
from pathlib import Path
from typing import Optional, Tuple

try:
    from kernel_craft_otel import kernel_span
except ImportError:  # the tracing module ships beside this one
    @contextlib.contextmanager
    def kernel_span(name, **attrs):
        yield None

# ---------------------------------------------------------------------------
# Loading the library
# ---------------------------------------------------------------------------


def _candidates() -> list:
    here = Path(__file__).resolve().parent
    found = [os.environ["KERNEL_CRAFT_LIB"]] if "KERNEL_CRAFT_LIB" in os.environ else []
    return found + [here.parent.parent / "build" / "libkernels.so",
                    here.parent.parent / "libkernels.so",
                    Path("/usr/local/lib/kernel_craft/libkernels.so")]


def _find_lib() -> str:
    """First existing libkernels.so in the discovery order; FileNotFoundError
    naming every place looked at otherwise."""
    paths = _candidates()
    for p in paths:
        if Path(p).exists():
            return str(p)
    raise FileNotFoundError("libkernels.so not found (build it with: make -C kernel-craft_amd); "
                            f"looked at {[str(p) for p in paths]}")


_LIB: Optional[ctypes.CDLL] = None


def _get_lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        lib = ctypes.CDLL(_find_lib(), mode=ctypes.RTLD_GLOBAL)
        _setup_prototypes(lib)
        _LIB = lib
    return _LIB


_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_b = ctypes.c_bool
_f = ctypes.c_float

# name -> (argtypes, restype).  The first seven are the symbols the
# reference binds at load time (reference :105-168).
PROTOTYPES = {
    "launch_flash_attention": ([_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _b, _vp], None),
    "launch_paged_attention": ([_vp] * 6 + [_i] * 6 + [_vp], None),
    "launch_dequantize_int4": ([_vp, _vp, _vp, _vp, _i, _i, _i, _vp], None),
    "launch_gemv_int4": ([_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp], None),
    "launch_quantize_fp8": ([_vp, _vp, _vp, _i, _i, _b, _vp], None),
    "launch_dequantize_fp8": ([_vp, _vp, _vp, _i, _i, _b, _vp], None),
    "launch_verify_draft_tokens": ([_vp] * 7 + [_i, _i, _vp], None),
    # further reference launchers, the error channel and the extensions
    "launch_smoothquant_scale": ([_vp, _vp, _vp, _i, _i, _vp], None),
    "launch_rmsnorm": ([_vp, _vp, _vp, _i, _i, _f, _vp], None),
    "kc_get_last_error": ([], _i),
    "kc_peek_last_error": ([], _i),
    "kc_last_error_string": ([], ctypes.c_char_p),
    "kc_version": ([], ctypes.c_char_p),
    "kc_gemv_int4_f32_async": ([_vp] * 5 + [_i, _i, _i, _vp], _i),
    "kc_gemv_int4_bf16": ([_vp] * 5 + [_i, _i, _i, _vp], _i),
    "kc_gemm_int4_bf16": ([_vp] * 5 + [_i, _i, _i, _i, _vp], _i),
    "kc_gemv_int4_bf16_chain": ([_vp, _i, _vp], _i),
    "kc_shuffled_int4_bytes": ([_i64, _i64], _i64),
    "kc_shuffle_int4_mfma": ([_vp, _vp, _i, _i, _vp], _i),
    "kc_gemm_int4_bf16_shuffled": ([_vp] * 5 + [_i, _i, _i, _i, _vp], _i),
    "kc_convert_gptq_int4": ([_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp], _i),
    "kc_convert_awq_int4": ([_vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp], _i),
    "kc_gemm_fp8_w8a8_bf16": ([_vp] * 5 + [_i64, _i64, _i64, _vp], _i),
    "kc_gemm_fp8_w8a8_f32": ([_vp] * 5 + [_i64, _i64, _i64, _vp], _i),
    "kc_quantize_fp8_per_token_f32": ([_vp, _vp, _vp, _i64, _i64, _vp], _i),
    "kc_quantize_fp8_per_tensor_f32": ([_vp, _vp, _vp, _i64, _i64, _vp], _i),
    "kc_quantize_fp8_per_token_bf16": ([_vp, _vp, _vp, _i64, _i64, _vp], _i),
    "kc_col_absmax_bf16": ([_vp, _vp, _i64, _i64, _vp], _i),
    "kc_col_absmax_f32": ([_vp, _vp, _i64, _i64, _vp], _i),
    "kc_smooth_factors": ([_vp, _vp, _vp, _i64, _vp], _i),
    "kc_smoothquant_stats_bf16": ([_vp, _i64, _vp, _i64, _i64, _vp, _vp, _vp, _vp], _i),
    "kc_smoothquant_stats_f32": ([_vp, _i64, _vp, _i64, _i64, _vp, _vp, _vp, _vp], _i),
    "kc_quantize_fp8_smooth_div_f32": ([_vp, _vp, _vp, _vp, _i64, _i64, _vp], _i),
    "kc_quantize_fp8_smooth_div_bf16": ([_vp, _vp, _vp, _vp, _i64, _i64, _vp], _i),
    "kc_quantize_fp8_smooth_mul_bf16": ([_vp, _vp, _vp, _vp, _i64, _i64, _vp], _i),
    "kc_rmsnorm_bf16": ([_vp, _vp, _vp, _i, _i, _f, _vp], _i),
    "kc_rmsnorm_gemv_int4_bf16": ([_vp, _vp, _f, _vp, _vp, _vp, _vp, _i, _i, _i, _vp], _i),
    "kc_rmsnorm_quantize_fp8_bf16": ([_vp, _vp, _f, _vp, _vp, _i64, _i64, _vp], _i),
}


def _setup_prototypes(lib: ctypes.CDLL) -> None:
    """Bind argtypes/restype of every symbol in PROTOTYPES (AttributeError
    for a symbol the library does not export)."""
    for name, (argtypes, restype) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype


# ---------------------------------------------------------------------------
# Arguments and errors
# ---------------------------------------------------------------------------


def _stream() -> ctypes.c_void_p:
    """The current torch stream (a hipStream_t) for the launchers."""
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t) -> ctypes.c_void_p:
    """Device address of a tensor's first element."""
    return ctypes.c_void_p(t.data_ptr())


def _arg(name: str, t, dtypes=None, numel: Optional[int] = None):
    """``t`` made contiguous after checking that it has one of ``dtypes``
    and holds at least ``numel`` elements (what the kernels read or write
    through it); ValueError otherwise.  Every op checks all of its arguments
    this way, then their device with ``_on_gpu``, before it allocates or
    launches anything."""
    if dtypes is not None:
        allowed = dtypes if isinstance(dtypes, tuple) else (dtypes,)
        if t.dtype not in allowed:
            raise ValueError(f"{name} has dtype {t.dtype}; expected "
                             f"{' or '.join(str(d) for d in allowed)}")
    if numel is not None and t.numel() < numel:
        raise ValueError(f"{name} holds {t.numel()} elements; the shape arguments need "
                         f"at least {numel}")
    return t.contiguous()


def _on_gpu(op: str, *tensors) -> None:
    """ValueError unless every tensor lives on a GPU."""
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError(f"{op}: a tensor is on {t.device}; kernel_craft ops run on the "
                             "GPU only (there is no CPU fallback)")


def _int4_meta(op: str, scales, zeros, rows: int, cols: int, group_size: int):
    """Validated (scales, zeros) of an INT4 layer [rows, cols]: scales [rows,
    G] fp32 and zero bytes read at row stride floor(G/2) (quant_int4.cu:93,
    152), so the last row reaches byte (rows-1)*floor(G/2) + (G-1)/2, with
    G = cols / group_size.  Bad shape arguments are left to the library,
    which rejects them with a message."""
    import torch
    ok = rows > 0 and cols > 0 and group_size > 0
    G = cols // group_size if ok else 0
    zneed = (rows - 1) * (G // 2) + (G - 1) // 2 + 1 if ok and G > 0 else 0
    return (_arg(f"{op}: scales", scales, torch.float32, rows * G if ok else None),
            _arg(f"{op}: zeros", zeros, torch.uint8, zneed))


def _int4_weights(op: str, packed, scales, zeros, rows: int, cols: int, group_size: int):
    """Validated (packed, scales, zeros) of an INT4 layer [rows, cols] in the
    reference layout: packed [rows, cols/2] u8, scales and zeros as
    _int4_meta checks them."""
    import torch
    ok = rows > 0 and cols > 0 and group_size > 0
    packed = _arg(f"{op}: packed", packed, torch.uint8, rows * (cols // 2) if ok else None)
    return (packed,) + _int4_meta(op, scales, zeros, rows, cols, group_size)


def _check(name: str, status: Optional[int] = None) -> None:
    """RuntimeError if the call returned a non-zero status or (void
    launchers) left an error in the library's channel; clears the channel."""
    lib = _get_lib()
    code = lib.kc_get_last_error()
    code = status or code
    if code:
        msg = lib.kc_last_error_string().decode(errors="replace")
        raise RuntimeError(f"{name} failed (kc_status {code}): {msg}")


def last_error() -> Tuple[int, str]:
    """(code, message) of the calling thread's last library error; clears it."""
    lib = _get_lib()
    msg = lib.kc_last_error_string().decode(errors="replace")
    return lib.kc_get_last_error(), msg


def _stub_op(op: str, symbol: str, span_attrs: dict, pointer_args, int_args):
    """An op whose launcher this build exports as a stub (outside the
    quantized-inference path): the call is made so that the library's
    not-implemented error surfaces as RuntimeError, inside the same span the
    reference opens for it."""
    with kernel_span(op, **span_attrs):
        getattr(_get_lib(), symbol)(*[_ptr(t) for t in pointer_args], *int_args, _stream())
    _check(op)


# ---------------------------------------------------------------------------
# The reference's operators (reference :193-421)
# ---------------------------------------------------------------------------


def flash_attention(Q, K, V, H_kv: int, causal: bool = False):
    """Prefill attention [B, H, N, d] (reference op; this library's launcher
    is a stub, so the call raises RuntimeError)."""
    import torch
    Q, K, V = (_arg("flash_attention: " + n, t, torch.float32) for n, t in
               (("Q", Q), ("K", K), ("V", V)))
    _on_gpu("flash_attention", Q, K, V)
    B, H, N, d = Q.shape
    out = torch.zeros(B, H, N, d, dtype=torch.float32, device=Q.device)
    _stub_op("flash_attention", "launch_flash_attention",
             dict(batch=B, heads=H, kv_heads=H_kv, seq_len=N, head_dim=d, causal=causal),
             (Q, K, V, out), (B, H, H_kv, N, d, causal))
    return out


def paged_attention(Q, block_table, K_pool, V_pool, seq_lens, H_kv: int, block_size: int):
    """Decode attention over a paged KV cache, output [B, H, d] (reference
    op; stub launcher, raises RuntimeError)."""
    import torch
    Q, K_pool, V_pool = (_arg("paged_attention: " + n, t, torch.float32) for n, t in
                         (("Q", Q), ("K_pool", K_pool), ("V_pool", V_pool)))
    block_table = _arg("paged_attention: block_table", block_table, torch.int32)
    seq_lens = _arg("paged_attention: seq_lens", seq_lens, torch.int32)
    _on_gpu("paged_attention", Q, block_table, K_pool, V_pool, seq_lens)
    B, H, d = Q.shape
    out = torch.zeros(B, H, d, dtype=torch.float32, device=Q.device)
    _stub_op("paged_attention", "launch_paged_attention",
             dict(batch=B, heads=H, kv_heads=H_kv, seq_len=int(seq_lens.max().item()),
                  block_size=block_size),
             (Q, block_table, K_pool, V_pool, out, seq_lens),
             (B, H, H_kv, d, block_size, block_table.shape[1]))
    return out


def speculative_verify(draft_probs, target_probs, draft_tokens, rand_vals, rand_vals2) -> Tuple:
    """Draft-token acceptance for speculative decoding, returning int32
    (accepted [K], corrected [K]) (reference op; stub launcher, raises
    RuntimeError)."""
    import torch
    draft_probs, target_probs, rand_vals, rand_vals2 = (
        _arg("speculative_verify: " + n, t, torch.float32) for n, t in
        (("draft_probs", draft_probs), ("target_probs", target_probs),
         ("rand_vals", rand_vals), ("rand_vals2", rand_vals2)))
    draft_tokens = _arg("speculative_verify: draft_tokens", draft_tokens, torch.int32)
    _on_gpu("speculative_verify", draft_probs, target_probs, draft_tokens, rand_vals, rand_vals2)
    K, vocab = draft_probs.shape
    accepted = torch.zeros(K, dtype=torch.int32, device=draft_probs.device)
    corrected = torch.zeros(K, dtype=torch.int32, device=draft_probs.device)
    _stub_op("speculative_verify", "launch_verify_draft_tokens",
             dict(num_tokens=K, vocab_size=vocab),
             (draft_probs, target_probs, draft_tokens, rand_vals, rand_vals2, accepted,
              corrected), (K, vocab))
    return accepted, corrected


def int4_dequantize(packed, scales, zeros, rows: int, cols: int, group_size: int = 128):
    """INT4 layer -> fp32 W [rows, cols], W[n, k] = (sext4(q) - z) * s
    (launch_dequantize_int4)."""
    import torch
    packed, scales, zeros = _int4_weights("int4_dequantize", packed, scales, zeros, rows, cols,
                                          group_size)
    _on_gpu("int4_dequantize", packed, scales, zeros)
    out = torch.zeros(rows, cols, dtype=torch.float32, device=packed.device)
    _get_lib().launch_dequantize_int4(_ptr(packed), _ptr(scales), _ptr(zeros), _ptr(out),
                                      rows, cols, group_size, _stream())
    _check("int4_dequantize")
    return out


def int4_gemv(packed, scales, zeros, x, rows: int, cols: int, group_size: int = 128):
    """y [rows] = W x for an INT4 layer and fp32 x [cols], fp32 accumulation
    (launch_gemv_int4)."""
    import torch
    packed, scales, zeros = _int4_weights("int4_gemv", packed, scales, zeros, rows, cols,
                                          group_size)
    x = _arg("int4_gemv: x", x, torch.float32, cols)
    _on_gpu("int4_gemv", packed, scales, zeros, x)
    y = torch.zeros(rows, dtype=torch.float32, device=packed.device)
    with kernel_span("int4_gemv", rows=rows, cols=cols, group_size=group_size):
        _get_lib().launch_gemv_int4(_ptr(packed), _ptr(scales), _ptr(zeros), _ptr(x), _ptr(y),
                                    rows, cols, group_size, _stream())
    _check("int4_gemv")
    return y


def fp8_quantize(x, per_token: bool = True) -> Tuple:
    """fp32 x [rows, cols] -> (int8 E4M3 codes [rows, cols], fp32 scales
    [rows] per token or [1]) (launch_quantize_fp8).

    Per-tensor mode reads its scale from the freshly zeroed scales buffer, as
    the reference bridge does (reference :345-347), so every code saturates
    to +-448."""
    import torch
    x = _arg("fp8_quantize: x", x, torch.float32)
    _on_gpu("fp8_quantize", x)
    rows, cols = x.shape
    q = torch.zeros(rows, cols, dtype=torch.int8, device=x.device)
    scales = torch.zeros(rows if per_token else 1, dtype=torch.float32, device=x.device)
    with kernel_span("fp8_quantize", rows=rows, cols=cols, per_token=per_token):
        _get_lib().launch_quantize_fp8(_ptr(x), _ptr(q), _ptr(scales), rows, cols, per_token,
                                       _stream())
    _check("fp8_quantize")
    return q, scales


def fp8_dequantize(q, scales, rows: int, cols: int, per_token: bool = True):
    """int8 E4M3 codes [rows, cols] and their scales -> fp32 [rows, cols]
    (launch_dequantize_fp8)."""
    import torch
    q = _arg("fp8_dequantize: q", q, (torch.int8, torch.uint8), rows * cols)
    scales = _arg("fp8_dequantize: scales", scales, torch.float32,
                  rows if per_token else None)
    if not per_token and scales.numel() < 1:
        raise ValueError("fp8_dequantize: per-tensor mode needs one scale")
    _on_gpu("fp8_dequantize", q, scales)
    out = torch.zeros(rows, cols, dtype=torch.float32, device=q.device)
    _get_lib().launch_dequantize_fp8(_ptr(q), _ptr(scales), _ptr(out), rows, cols, per_token,
                                     _stream())
    _check("fp8_dequantize")
    return out


# ---------------------------------------------------------------------------
# Extensions (no reference counterpart)
# ---------------------------------------------------------------------------


def smoothquant_scale(x, smooth_scales):
    """out[r, c] = x[r, c] / smooth_scales[c], fp32 (launch_smoothquant_scale)."""
    import torch
    x = _arg("smoothquant_scale: x", x, torch.float32)
    rows, cols = x.shape
    smooth_scales = _arg("smoothquant_scale: smooth_scales", smooth_scales, torch.float32, cols)
    _on_gpu("smoothquant_scale", x, smooth_scales)
    out = torch.zeros(rows, cols, dtype=torch.float32, device=x.device)
    _get_lib().launch_smoothquant_scale(_ptr(x), _ptr(smooth_scales), _ptr(out), rows, cols,
                                        _stream())
    _check("smoothquant_scale")
    return out


def int4_gemv_bf16(packed, scales, zeros, x, rows: int, cols: int, group_size: int = 128):
    """y [rows] bf16 = W x for bf16 x [cols], fp32 accumulation (kc_gemv_int4_bf16)."""
    import torch
    packed, scales, zeros = _int4_weights("int4_gemv_bf16", packed, scales, zeros, rows, cols,
                                          group_size)
    x = _arg("int4_gemv_bf16: x", x, torch.bfloat16, cols)
    _on_gpu("int4_gemv_bf16", packed, scales, zeros, x)
    y = torch.empty(rows, dtype=torch.bfloat16, device=packed.device)
    with kernel_span("int4_gemv_bf16", rows=rows, cols=cols, group_size=group_size):
        st = _get_lib().kc_gemv_int4_bf16(_ptr(packed), _ptr(scales), _ptr(zeros), _ptr(x),
                                          _ptr(y), rows, cols, group_size, _stream())
    _check("int4_gemv_bf16", st)
    return y


class GemvOp(ctypes.Structure):
    """kc_gemv_op (include/kernel_craft.h): one GEMV of a chain."""
    _fields_ = [("packed", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("zeros", ctypes.c_void_p), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("rows", ctypes.c_int), ("cols", ctypes.c_int), ("group_size", ctypes.c_int),
                ("reserved", ctypes.c_int)]


def int4_gemv_bf16_chain(ops) -> None:
    """int4_gemv_bf16 for each op in order, from one call.  ``ops`` is a list
    of (packed, scales, zeros, x, y, rows, cols, group_size) with bf16 x and y
    already allocated and contiguous (the op writes into y, so a copy would
    lose the result); an op's x may be an earlier op's y or a contiguous
    slice of it.

    Weights that are not contiguous are copied first; every copy is held in
    ``keep`` until the library call has returned, so no op points at memory
    the caching allocator has handed to a later copy.  The kernels run
    asynchronously on the current stream, which orders the copies' eventual
    reuse after them.  A caller that captures this call in a HIP graph must
    pass contiguous weights: the graph keeps the pointers, not the copies."""
    import torch
    arr = (GemvOp * max(1, len(ops)))()
    keep = []
    for i, (packed, scales, zeros, x, y, rows, cols, gs) in enumerate(ops):
        name = f"int4_gemv_bf16_chain op {i}"
        if not (x.is_contiguous() and y.is_contiguous()):
            raise ValueError(f"{name}: x and y must be contiguous")
        packed, scales, zeros = _int4_weights(name, packed, scales, zeros, rows, cols, gs)
        _arg(f"{name}: x", x, torch.bfloat16, cols)
        _arg(f"{name}: y", y, torch.bfloat16, rows)
        _on_gpu(name, packed, scales, zeros, x, y)
        keep.append((packed, scales, zeros))
        arr[i] = GemvOp(_ptr(packed), _ptr(scales), _ptr(zeros), _ptr(x), _ptr(y), rows, cols,
                        gs, 0)
    with kernel_span("int4_gemv_bf16_chain", ops=len(ops)):
        st = _get_lib().kc_gemv_int4_bf16_chain(ctypes.cast(arr, ctypes.c_void_p), len(ops),
                                                _stream())
    _check("int4_gemv_bf16_chain", st)
    del keep


def int4_gemm_bf16(packed, scales, zeros, x, rows: int, cols: int, group_size: int = 128):
    """Y [m, rows] bf16 = X W^T for bf16 X [m, cols], 1 <= m <= 64, on matrix
    cores (kc_gemm_int4_bf16)."""
    import torch
    packed, scales, zeros = _int4_weights("int4_gemm_bf16", packed, scales, zeros, rows, cols,
                                          group_size)
    x = _arg("int4_gemm_bf16: x", x, torch.bfloat16)
    if x.dim() != 2 or x.shape[1] != cols:
        raise ValueError(f"int4_gemm_bf16: x must be [m, {cols}], not {list(x.shape)}")
    _on_gpu("int4_gemm_bf16", packed, scales, zeros, x)
    m = x.shape[0]
    y = torch.empty(m, rows, dtype=torch.bfloat16, device=packed.device)
    with kernel_span("int4_gemm_bf16", m=m, rows=rows, cols=cols, group_size=group_size):
        st = _get_lib().kc_gemm_int4_bf16(_ptr(packed), _ptr(scales), _ptr(zeros), _ptr(x),
                                          _ptr(y), m, rows, cols, group_size, _stream())
    _check("int4_gemm_bf16", st)
    return y


def int4_shuffle_mfma(packed, rows: int, cols: int):
    """The pre-shuffled layout of packed [rows, cols/2] u8 for the matrix-core
    kernels (kc_shuffle_int4_mfma): a u8 vector of ceil(rows/16)*16*cols/2
    bytes.  cols must be a multiple of 128; scales and zeros stay as they are."""
    import torch
    nbytes = _get_lib().kc_shuffled_int4_bytes(rows, cols)
    if nbytes < 0 or rows < 0:
        raise ValueError(f"int4_shuffle_mfma: rows={rows} cols={cols} (cols must be a multiple of 128)")
    packed = _arg("int4_shuffle_mfma: packed", packed, torch.uint8, rows * (cols // 2))
    _on_gpu("int4_shuffle_mfma", packed)
    out = torch.empty(nbytes, dtype=torch.uint8, device=packed.device)
    with kernel_span("int4_shuffle_mfma", rows=rows, cols=cols):
        st = _get_lib().kc_shuffle_int4_mfma(_ptr(packed), _ptr(out), rows, cols, _stream())
    _check("int4_shuffle_mfma", st)
    return out


def int4_gemm_bf16_shuffled(packed_shuffled, scales, zeros, x, rows: int, cols: int,
                            group_size: int = 128):
    """int4_gemm_bf16 on weights in the shuffled layout (int4_shuffle_mfma):
    Y [m, rows] bf16 for bf16 X [m, cols], 1 <= m <= 64
    (kc_gemm_int4_bf16_shuffled)."""
    import torch
    nbytes = _get_lib().kc_shuffled_int4_bytes(rows, cols)
    if nbytes < 0 or rows < 0:
        raise ValueError(f"int4_gemm_bf16_shuffled: rows={rows} cols={cols} (cols must be a "
                         "multiple of 128)")
    packed_shuffled = _arg("int4_gemm_bf16_shuffled: packed_shuffled", packed_shuffled, torch.uint8,
                           nbytes)
    scales, zeros = _int4_meta("int4_gemm_bf16_shuffled", scales, zeros, rows, cols, group_size)
    x = _arg("int4_gemm_bf16_shuffled: x", x, torch.bfloat16)
    if x.dim() != 2 or x.shape[1] != cols:
        raise ValueError(f"int4_gemm_bf16_shuffled: x must be [m, {cols}], not {list(x.shape)}")
    _on_gpu("int4_gemm_bf16_shuffled", packed_shuffled, scales, zeros, x)
    m = x.shape[0]
    y = torch.empty(m, rows, dtype=torch.bfloat16, device=packed_shuffled.device)
    with kernel_span("int4_gemm_bf16_shuffled", m=m, rows=rows, cols=cols, group_size=group_size):
        st = _get_lib().kc_gemm_int4_bf16_shuffled(_ptr(packed_shuffled), _ptr(scales), _ptr(zeros),
                                                   _ptr(x), _ptr(y), m, rows, cols, group_size,
                                                   _stream())
    _check("int4_gemm_bf16_shuffled", st)
    return y


def act_order_permutation(g_idx, group_size: int):
    """The input-channel order that makes an act-order GPTQ checkpoint's
    groups contiguous: a stable sort of k by g_idx, checked to give every
    group exactly group_size channels.  None when g_idx is already k //
    group_size."""
    import torch
    g = g_idx.detach().to("cpu", torch.int64).reshape(-1)
    K = g.numel()
    if K % group_size:
        raise ValueError(f"g_idx has {K} entries, not a multiple of group_size={group_size}")
    if torch.equal(g, torch.arange(K) // group_size):
        return None
    counts = torch.bincount(g, minlength=K // group_size)
    if counts.numel() != K // group_size or not bool((counts == group_size).all()):
        raise ValueError("g_idx does not give every group exactly group_size input channels")
    return torch.sort(g, stable=True).indices.to(torch.int32)


def convert_gptq(qweight, qzeros, scales, g_idx=None, group_size: int = 128, zero_offset: int = 1):
    """A GPTQ checkpoint layer (qweight int32 [K/8, N], qzeros int32 [G, N/8],
    scales fp16 [G, N], optional g_idx [K]) to the reference layout:
    returns (packed u8 [N, K/2], scales fp32 [N, G], zeros u8 [N, G/2], perm).
    perm is None, or an int32 [K] tensor: the converted weights expect
    x[perm] (act-order checkpoints).  zero_offset is 1 for the original
    AutoGPTQ format (zero points stored minus one), 0 for its v2."""
    import torch
    qweight = _arg("convert_gptq: qweight", qweight, torch.int32)
    K, N = qweight.shape[0] * 8, qweight.shape[1]
    G = K // group_size if group_size > 0 else 0
    qzeros = _arg("convert_gptq: qzeros", qzeros, torch.int32, G * (N // 8))
    scales = _arg("convert_gptq: scales", scales, torch.float16, G * N)
    _on_gpu("convert_gptq", qweight, qzeros, scales)
    perm = None if g_idx is None else act_order_permutation(g_idx, group_size)
    dperm = None if perm is None else perm.to(qweight.device)
    packed = torch.empty(N, K // 2, dtype=torch.uint8, device=qweight.device)
    out_s = torch.empty(N, G, dtype=torch.float32, device=qweight.device)
    zeros = torch.empty(N, G // 2, dtype=torch.uint8, device=qweight.device)
    with kernel_span("convert_gptq", rows=N, cols=K, group_size=group_size):
        st = _get_lib().kc_convert_gptq_int4(_ptr(qweight), _ptr(qzeros), _ptr(scales),
                                             _ptr(dperm) if dperm is not None else None,
                                             K, N, group_size, zero_offset, _ptr(packed),
                                             _ptr(out_s), _ptr(zeros), _stream())
    _check("convert_gptq", st)
    return packed, out_s, zeros, dperm


def convert_awq(qweight, qzeros, scales, group_size: int = 128):
    """An AWQ (GEMM-format) layer (qweight int32 [K, N/8], qzeros int32
    [G, N/8], scales fp16 [G, N]) to the reference layout: returns (packed
    u8 [N, K/2], scales fp32 [N, G], zeros u8 [N, G/2])."""
    import torch
    qweight = _arg("convert_awq: qweight", qweight, torch.int32)
    K, N = qweight.shape[0], qweight.shape[1] * 8
    G = K // group_size if group_size > 0 else 0
    qzeros = _arg("convert_awq: qzeros", qzeros, torch.int32, G * (N // 8))
    scales = _arg("convert_awq: scales", scales, torch.float16, G * N)
    _on_gpu("convert_awq", qweight, qzeros, scales)
    packed = torch.empty(N, K // 2, dtype=torch.uint8, device=qweight.device)
    out_s = torch.empty(N, G, dtype=torch.float32, device=qweight.device)
    zeros = torch.empty(N, G // 2, dtype=torch.uint8, device=qweight.device)
    with kernel_span("convert_awq", rows=N, cols=K, group_size=group_size):
        st = _get_lib().kc_convert_awq_int4(_ptr(qweight), _ptr(qzeros), _ptr(scales), K, N,
                                            group_size, _ptr(packed), _ptr(out_s), _ptr(zeros),
                                            _stream())
    _check("convert_awq", st)
    return packed, out_s, zeros


def fp8_gemm_w8a8(qx, sx, qw, sw, out_dtype=None):
    """Y [M, N] = sx[m] sw[n] sum_k e4m3(qx[m,k]) e4m3(qw[n,k]) on FP8 matrix
    cores: qx int8 [M, K] / sx fp32 [M] from fp8_quantize_rows on the
    activations, qw int8 [N, K] / sw fp32 [N] from it on the weights.
    out_dtype torch.bfloat16 (default) or torch.float32."""
    import torch
    out_dtype = torch.bfloat16 if out_dtype is None else out_dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"fp8_gemm_w8a8: out_dtype must be bfloat16 or float32, not {out_dtype}")
    qx = _arg("fp8_gemm_w8a8: qx", qx, (torch.int8, torch.uint8))
    qw = _arg("fp8_gemm_w8a8: qw", qw, (torch.int8, torch.uint8))
    if qx.dim() != 2 or qw.dim() != 2 or qw.shape[1] != qx.shape[1]:
        raise ValueError("fp8_gemm_w8a8: qx [M, K] and qw [N, K] must share K")
    M, K = qx.shape
    N = qw.shape[0]
    sx = _arg("fp8_gemm_w8a8: sx", sx, torch.float32, M)
    sw = _arg("fp8_gemm_w8a8: sw", sw, torch.float32, N)
    _on_gpu("fp8_gemm_w8a8", qx, sx, qw, sw)
    y = torch.empty(M, N, dtype=out_dtype, device=qx.device)
    fn = (_get_lib().kc_gemm_fp8_w8a8_bf16 if out_dtype == torch.bfloat16
          else _get_lib().kc_gemm_fp8_w8a8_f32)
    with kernel_span("fp8_gemm_w8a8", m=M, n=N, k=K):
        st = fn(_ptr(qx), _ptr(sx), _ptr(qw), _ptr(sw), _ptr(y), M, N, K, _stream())
    _check("fp8_gemm_w8a8", st)
    return y


def rmsnorm(x, g, eps: float = 1e-6):
    """y = g * x / sqrt(mean(x^2, -1) + eps) per row (rmsnorm.cu:40-70):
    fp32 x and g through launch_rmsnorm, bf16 through kc_rmsnorm_bf16."""
    import torch
    x = _arg("rmsnorm: x", x, (torch.float32, torch.bfloat16))
    D = x.shape[-1]
    rows = x.numel() // max(D, 1)
    g = _arg("rmsnorm: g", g, x.dtype, D)
    _on_gpu("rmsnorm", x, g)
    y = torch.empty_like(x)
    with kernel_span("rmsnorm", rows=rows, d=D):
        if x.dtype == torch.float32:
            _get_lib().launch_rmsnorm(_ptr(x), _ptr(g), _ptr(y), rows, D, eps, _stream())
            st = None
        else:
            st = _get_lib().kc_rmsnorm_bf16(_ptr(x), _ptr(g), _ptr(y), rows, D, eps, _stream())
    _check("rmsnorm", st)
    return y


def rmsnorm_int4_gemv_bf16(h, gamma, packed, scales, zeros, rows: int, cols: int,
                           group_size: int = 128, eps: float = 1e-6):
    """y = W_int4 * bf16(rmsnorm(h) * gamma) in one launch: bf16 h, gamma
    [cols], bf16 y [rows] (kc_rmsnorm_gemv_int4_bf16)."""
    import torch
    packed, scales, zeros = _int4_weights("rmsnorm_int4_gemv_bf16", packed, scales, zeros, rows,
                                          cols, group_size)
    h = _arg("rmsnorm_int4_gemv_bf16: h", h, torch.bfloat16, cols)
    gamma = _arg("rmsnorm_int4_gemv_bf16: gamma", gamma, torch.bfloat16, cols)
    _on_gpu("rmsnorm_int4_gemv_bf16", h, gamma, packed, scales, zeros)
    y = torch.empty(rows, dtype=torch.bfloat16, device=packed.device)
    with kernel_span("rmsnorm_int4_gemv_bf16", rows=rows, cols=cols, group_size=group_size):
        st = _get_lib().kc_rmsnorm_gemv_int4_bf16(_ptr(h), _ptr(gamma), eps, _ptr(packed),
                                                  _ptr(scales), _ptr(zeros), _ptr(y), rows, cols,
                                                  group_size, _stream())
    _check("rmsnorm_int4_gemv_bf16", st)
    return y


def rmsnorm_fp8_quantize(h, gamma, eps: float = 1e-6) -> Tuple:
    """RMSNorm of bf16 h [T, D] with bf16 gamma [D], quantized per token to
    FP8 in one pass: (int8 codes [T, D], fp32 scales [T]), the same bits as
    fp8_quantize_rows(rmsnorm(h, gamma, eps)) (kc_rmsnorm_quantize_fp8_bf16)."""
    import torch
    h = _arg("rmsnorm_fp8_quantize: h", h, torch.bfloat16)
    if h.dim() != 2:
        raise ValueError("rmsnorm_fp8_quantize: h must be [T, D]")
    T, D = h.shape
    gamma = _arg("rmsnorm_fp8_quantize: gamma", gamma, torch.bfloat16, D)
    _on_gpu("rmsnorm_fp8_quantize", h, gamma)
    q = torch.empty(T, D, dtype=torch.int8, device=h.device)
    # an empty row has absmax 0, hence scale 1; the library writes nothing
    # when D == 0 (as the reference launcher, whose launch has no threads)
    s = (torch.ones if D == 0 else torch.empty)(T, dtype=torch.float32, device=h.device)
    with kernel_span("rmsnorm_fp8_quantize", rows=T, cols=D):
        st = _get_lib().kc_rmsnorm_quantize_fp8_bf16(_ptr(h), _ptr(gamma), eps, _ptr(q), _ptr(s),
                                                     T, D, _stream())
    _check("rmsnorm_fp8_quantize", st)
    return q, s


def fp8_quantize_rows(x) -> Tuple:
    """Per-row FP8 quantization of a bf16 or fp32 [rows, cols] tensor: per
    token for activations, per output channel for a weight matrix."""
    import torch
    x = _arg("fp8_quantize_rows: x", x, (torch.float32, torch.bfloat16))
    _on_gpu("fp8_quantize_rows", x)
    rows, cols = x.shape
    q = torch.empty(rows, cols, dtype=torch.int8, device=x.device)
    # scale 1 for empty rows (absmax 0), which the library does not write
    s = (torch.ones if cols == 0 else torch.empty)(rows, dtype=torch.float32, device=x.device)
    lib = _get_lib()
    fn = lib.kc_quantize_fp8_per_token_bf16 if x.dtype == torch.bfloat16 \
        else lib.kc_quantize_fp8_per_token_f32
    with kernel_span("fp8_quantize_rows", rows=rows, cols=cols, dtype=str(x.dtype)):
        st = fn(_ptr(x), _ptr(q), _ptr(s), rows, cols, _stream())
    _check("fp8_quantize_rows", st)
    return q, s


def col_absmax(x):
    """Per-column max |x| of a bf16 or fp32 [rows, cols] tensor."""
    import torch
    x = _arg("col_absmax: x", x, (torch.float32, torch.bfloat16))
    _on_gpu("col_absmax", x)
    rows, cols = x.shape
    out = torch.empty(cols, dtype=torch.float32, device=x.device)
    lib = _get_lib()
    fn = lib.kc_col_absmax_bf16 if x.dtype == torch.bfloat16 else lib.kc_col_absmax_f32
    st = fn(_ptr(x), _ptr(out), rows, cols, _stream())
    _check("col_absmax", st)
    return out


def smooth_factors(amax_x, amax_w):
    """SmoothQuant factors (alpha = 0.5) from per-channel absmax of X and W."""
    import torch
    amax_x = _arg("smooth_factors: amax_x", amax_x, torch.float32)
    amax_w = _arg("smooth_factors: amax_w", amax_w, torch.float32, amax_x.numel())
    _on_gpu("smooth_factors", amax_x, amax_w)
    s = torch.empty_like(amax_x)
    st = _get_lib().kc_smooth_factors(_ptr(amax_x), _ptr(amax_w), _ptr(s), amax_x.numel(),
                                      _stream())
    _check("smooth_factors", st)
    return s


def smoothquant_stats(x, w) -> Tuple:
    """SmoothQuant statistics of activations x [tokens, cols] and weights
    w [out_features, cols] (both bf16 or both fp32) in one library call:
    (amax_x, amax_w, smooth), the values col_absmax(x), col_absmax(w) and
    smooth_factors give."""
    import torch
    x = _arg("smoothquant_stats: x", x, (torch.float32, torch.bfloat16))
    w = _arg("smoothquant_stats: w", w, x.dtype)
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise ValueError(f"smoothquant_stats: x {tuple(x.shape)} and w {tuple(w.shape)} must be "
                         "2-D with the same number of columns")
    _on_gpu("smoothquant_stats", x, w)
    cols = x.shape[1]
    amax_x = torch.empty(cols, dtype=torch.float32, device=x.device)
    amax_w = torch.empty_like(amax_x)
    s = torch.empty_like(amax_x)
    lib = _get_lib()
    fn = lib.kc_smoothquant_stats_bf16 if x.dtype == torch.bfloat16 else lib.kc_smoothquant_stats_f32
    with kernel_span("smoothquant_stats", tokens=x.shape[0], out_features=w.shape[0], cols=cols):
        st = fn(_ptr(x), x.shape[0], _ptr(w), w.shape[0], cols, _ptr(amax_x), _ptr(amax_w), _ptr(s),
                _stream())
    _check("smoothquant_stats", st)
    return amax_x, amax_w, s


def fp8_quantize_smooth(x, smooth, mode: str = "div") -> Tuple:
    """Fused SmoothQuant + per-row FP8: ``div`` quantizes x / s (activations),
    ``mul`` quantizes x * s (weights, bf16 only)."""
    import torch
    if mode not in ("div", "mul"):
        raise ValueError(f"mode must be 'div' or 'mul', not {mode!r}")
    x = _arg("fp8_quantize_smooth: x", x,
             (torch.float32, torch.bfloat16) if mode == "div" else torch.bfloat16)
    rows, cols = x.shape
    smooth = _arg("fp8_quantize_smooth: smooth", smooth, torch.float32, cols)
    _on_gpu("fp8_quantize_smooth", x, smooth)
    q = torch.empty(rows, cols, dtype=torch.int8, device=x.device)
    s = torch.empty(rows, dtype=torch.float32, device=x.device)
    lib = _get_lib()
    if mode == "div":
        fn = lib.kc_quantize_fp8_smooth_div_bf16 if x.dtype == torch.bfloat16 \
            else lib.kc_quantize_fp8_smooth_div_f32
    else:
        fn = lib.kc_quantize_fp8_smooth_mul_bf16
    with kernel_span("fp8_quantize_smooth", rows=rows, cols=cols, mode=mode):
        st = fn(_ptr(x), _ptr(smooth), _ptr(q), _ptr(s), rows, cols, _stream())
    _check("fp8_quantize_smooth", st)
    return q, s


# ---------------------------------------------------------------------------
# torch.ops.kernel_craft (reference :428-479)
# ---------------------------------------------------------------------------

SCHEMAS = {
    "flash_attention": "flash_attention(Tensor Q, Tensor K, Tensor V, int H_kv, bool causal) -> Tensor",
    "paged_attention": ("paged_attention(Tensor Q, Tensor block_table, Tensor K_pool, "
                        "Tensor V_pool, Tensor seq_lens, int H_kv, int block_size) -> Tensor"),
    "int4_dequantize": ("int4_dequantize(Tensor packed, Tensor scales, Tensor zeros, "
                        "int rows, int cols, int group_size) -> Tensor"),
    "int4_gemv": ("int4_gemv(Tensor packed, Tensor scales, Tensor zeros, "
                  "Tensor x, int rows, int cols, int group_size) -> Tensor"),
    "fp8_quantize": "fp8_quantize(Tensor x, bool per_token) -> (Tensor, Tensor)",
    "fp8_dequantize": ("fp8_dequantize(Tensor q, Tensor scales, int rows, int cols, "
                       "bool per_token) -> Tensor"),
    "speculative_verify": ("speculative_verify(Tensor draft_probs, Tensor target_probs, "
                           "Tensor draft_tokens, Tensor rand_vals, Tensor rand_vals2) "
                           "-> (Tensor, Tensor)"),
}


def _register_torch_library() -> None:
    """Define SCHEMAS under torch.ops.kernel_craft and bind each to the
    function of the same name for the CPU and CUDA dispatch keys (CPU
    tensors then fail the device check inside the op).  The Library objects
    are kept in module globals: dropping them would unregister the ops."""
    import torch

    defs = torch.library.Library("kernel_craft", "DEF")
    impls = torch.library.Library("kernel_craft", "IMPL")
    ops = globals()
    for name, schema in SCHEMAS.items():
        defs.define(schema)
        for key in ("CPU", "CUDA"):
            impls.impl(name, ops[name], key)
    ops["_torch_lib_def"] = defs
    ops["_torch_lib_impl"] = impls


try:
    import torch  # noqa: F401
    _register_torch_library()
    TORCH_OPS_REGISTERED = True
except Exception:
    TORCH_OPS_REGISTERED = False
