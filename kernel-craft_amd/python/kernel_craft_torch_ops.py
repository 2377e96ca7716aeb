"""
kernel_craft_torch_ops.py
PyTorch operators over libkernels.so, the MI355X (gfx950) HIP build of
kernel-craft's quantized-inference kernels, loaded through ctypes.

This module keeps the reference bridge's interface
(``src/python/kernel_craft_torch_ops.py`` in kernel-craft): the same library
discovery order (``KERNEL_CRAFT_LIB``, ``../../build/libkernels.so``,
``../../libkernels.so``, ``/usr/local/lib/kernel_craft/libkernels.so``,
reference :68-87), ``RTLD_GLOBAL`` loading (:96), the same ctypes prototypes
(:101-168), the same public functions with the same arguments, output
allocations and OTEL span names/attributes (:265-381), and the same
``torch.library`` schema strings under the ``kernel_craft`` namespace
(:428-479).  On ROCm PyTorch, GPU tensors are ``device.type == "cuda"`` and
``torch.cuda.current_stream().cuda_stream`` is a ``hipStream_t``.

Differences from the reference, all of them additions:

* after every launcher call the library's error channel
  (``kc_get_last_error``) is read and a ``RuntimeError`` raised on failure,
  where the reference silently returns whatever the output buffer holds;
* inputs must live on a GPU: there is no CPU fallback, and a CPU tensor
  raises ``ValueError`` instead of handing a host pointer to a kernel;
* extra operators for the paths the reference lacks (bf16 GEMV, the M>1
  MFMA GEMM, bf16 FP8 quantization and fused SmoothQuant).

Usage
-----
::

    import kernel_craft_torch_ops as kc_ops
    y = kc_ops.int4_gemv(packed, scales, zeros, x, rows, cols, group_size=128)
    q, scales = kc_ops.fp8_quantize(x, per_token=True)
    x_hat     = kc_ops.fp8_dequantize(q, scales, rows, cols, per_token=True)

Building libkernels.so
----------------------
::

    make -C kernel-craft_amd          # produces build/libkernels.so
"""

import ctypes
import os
from pathlib import Path
from typing import Optional, Tuple

try:
    from kernel_craft_otel import kernel_span
except ImportError:  # pragma: no cover - the OTEL module ships beside this one
    from contextlib import nullcontext as kernel_span

# ---------------------------------------------------------------------------
# Library discovery (reference :68-87)
# ---------------------------------------------------------------------------


def _find_lib() -> str:
    """Return path to libkernels.so, searching standard locations."""
    candidates = []
    if "KERNEL_CRAFT_LIB" in os.environ:
        candidates.append(os.environ["KERNEL_CRAFT_LIB"])
    here = Path(__file__).resolve().parent
    candidates += [
        here.parent.parent / "build" / "libkernels.so",
        here.parent.parent / "libkernels.so",
        Path("/usr/local/lib/kernel_craft/libkernels.so"),
    ]
    for p in candidates:
        if Path(p).exists():
            return str(p)
    raise FileNotFoundError(
        "libkernels.so not found. Build with: make -C kernel-craft_amd\n"
        f"Searched: {[str(c) for c in candidates]}"
    )


_LIB: Optional[ctypes.CDLL] = None


def _get_lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = ctypes.CDLL(_find_lib(), mode=ctypes.RTLD_GLOBAL)
        _setup_prototypes(_LIB)
    return _LIB


_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_b = ctypes.c_bool

# name -> (argtypes, restype).  The first seven are the reference's own
# prototypes (reference :105-168); the reference binds them all at load time,
# so a missing symbol fails every op, exactly as there.
PROTOTYPES = {
    "launch_flash_attention": ([_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _b, _vp], None),
    "launch_paged_attention": ([_vp] * 6 + [_i] * 6 + [_vp], None),
    "launch_dequantize_int4": ([_vp, _vp, _vp, _vp, _i, _i, _i, _vp], None),
    "launch_gemv_int4": ([_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp], None),
    "launch_quantize_fp8": ([_vp, _vp, _vp, _i, _i, _b, _vp], None),
    "launch_dequantize_fp8": ([_vp, _vp, _vp, _i, _i, _b, _vp], None),
    "launch_verify_draft_tokens": ([_vp] * 7 + [_i, _i, _vp], None),
    # error channel and extensions (no reference counterpart)
    "launch_smoothquant_scale": ([_vp, _vp, _vp, _i, _i, _vp], None),
    "kc_get_last_error": ([], _i),
    "kc_peek_last_error": ([], _i),
    "kc_last_error_string": ([], ctypes.c_char_p),
    "kc_version": ([], ctypes.c_char_p),
    "kc_gemv_int4_f32_async": ([_vp] * 5 + [_i, _i, _i, _vp], _i),
    "kc_gemv_int4_bf16": ([_vp] * 5 + [_i, _i, _i, _vp], _i),
    "kc_gemm_int4_bf16": ([_vp] * 5 + [_i, _i, _i, _i, _vp], _i),
    "kc_gemv_int4_bf16_chain": ([_vp, _i, _vp], _i),
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
    "kc_quantize_fp8_smooth_div_f32": ([_vp, _vp, _vp, _vp, _i64, _i64, _vp], _i),
    "kc_quantize_fp8_smooth_div_bf16": ([_vp, _vp, _vp, _vp, _i64, _i64, _vp], _i),
    "kc_quantize_fp8_smooth_mul_bf16": ([_vp, _vp, _vp, _vp, _i64, _i64, _vp], _i),
    "launch_rmsnorm": ([_vp, _vp, _vp, _i, _i, ctypes.c_float, _vp], None),
    "kc_rmsnorm_bf16": ([_vp, _vp, _vp, _i, _i, ctypes.c_float, _vp], _i),
    "kc_rmsnorm_gemv_int4_bf16": ([_vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp, _i, _i, _i, _vp], _i),
}


def _setup_prototypes(lib: ctypes.CDLL) -> None:
    """Set ctypes argtypes/restype for every launcher."""
    for name, (argtypes, restype) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype


# ---------------------------------------------------------------------------
# Helpers
# ---------------------------------------------------------------------------


def _stream() -> ctypes.c_void_p:
    """Return the current HIP stream as a ctypes void pointer."""
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t) -> ctypes.c_void_p:
    """Return data_ptr of a torch tensor as ctypes void pointer."""
    return ctypes.c_void_p(t.data_ptr())


def _on_gpu(*tensors) -> None:
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError(
                "kernel_craft ops run on the GPU only; got a tensor on "
                f"{t.device} (there is no CPU fallback)")


def _check(name: str, status: Optional[int] = None) -> None:
    """Raise if the call recorded an error (void launchers) or returned one."""
    lib = _get_lib()
    code = lib.kc_get_last_error()
    if status:
        code = status
    if code:
        msg = lib.kc_last_error_string().decode(errors="replace")
        raise RuntimeError(f"{name} failed (kc_status {code}): {msg}")


def last_error() -> Tuple[int, str]:
    """(code, message) of the calling thread's last library error; clears it."""
    lib = _get_lib()
    msg = lib.kc_last_error_string().decode(errors="replace")
    return lib.kc_get_last_error(), msg


# ---------------------------------------------------------------------------
# Public API -- the reference's operators (reference :193-421)
# ---------------------------------------------------------------------------


def flash_attention(Q, K, V, H_kv: int, causal: bool = False):
    """FlashAttention prefill: out of scope for this build; the library's
    launcher is a stub that reports KC_ERR_NOT_IMPLEMENTED."""
    import torch
    Q, K, V = Q.contiguous(), K.contiguous(), V.contiguous()
    _on_gpu(Q, K, V)
    B, H, N, d = Q.shape
    O = torch.zeros(B, H, N, d, dtype=torch.float32, device=Q.device)
    with kernel_span("flash_attention", batch=B, heads=H, kv_heads=H_kv,
                     seq_len=N, head_dim=d, causal=causal):
        _get_lib().launch_flash_attention(
            _ptr(Q), _ptr(K), _ptr(V), _ptr(O), B, H, H_kv, N, d, causal, _stream())
    _check("flash_attention")
    return O


def paged_attention(Q, block_table, K_pool, V_pool, seq_lens, H_kv: int, block_size: int):
    """PagedAttention decode: out of scope for this build (stub launcher)."""
    import torch
    Q, block_table = Q.contiguous(), block_table.contiguous()
    K_pool, V_pool, seq_lens = K_pool.contiguous(), V_pool.contiguous(), seq_lens.contiguous()
    _on_gpu(Q, block_table, K_pool, V_pool, seq_lens)
    B, H, d = Q.shape
    max_blocks = block_table.shape[1]
    O = torch.zeros(B, H, d, dtype=torch.float32, device=Q.device)
    with kernel_span("paged_attention", batch=B, heads=H, kv_heads=H_kv,
                     seq_len=int(seq_lens.max().item()), block_size=block_size):
        _get_lib().launch_paged_attention(
            _ptr(Q), _ptr(block_table), _ptr(K_pool), _ptr(V_pool), _ptr(O), _ptr(seq_lens),
            B, H, H_kv, d, block_size, max_blocks, _stream())
    _check("paged_attention")
    return O


def int4_dequantize(packed, scales, zeros, rows: int, cols: int, group_size: int = 128):
    """
    Dequantize INT4 packed weights to FP32.

    :param packed     torch.Tensor [rows, cols/2] uint8 GPU
    :param scales     torch.Tensor [rows, cols/group_size] float32 GPU
    :param zeros      torch.Tensor [rows, cols/group_size/2] uint8 GPU
    :return:          torch.Tensor [rows, cols] float32 GPU
    """
    import torch
    packed, scales, zeros = packed.contiguous(), scales.contiguous(), zeros.contiguous()
    _on_gpu(packed, scales, zeros)
    output = torch.zeros(rows, cols, dtype=torch.float32, device=packed.device)
    _get_lib().launch_dequantize_int4(
        _ptr(packed), _ptr(scales), _ptr(zeros), _ptr(output), rows, cols, group_size, _stream())
    _check("int4_dequantize")
    return output


def int4_gemv(packed, scales, zeros, x, rows: int, cols: int, group_size: int = 128):
    """
    INT4 weight GEMV: y = W_int4 * x (dequantize on the fly).

    :param x          torch.Tensor [cols] float32 GPU
    :return:          torch.Tensor [rows] float32 GPU
    """
    import torch
    packed, scales, zeros, x = (packed.contiguous(), scales.contiguous(),
                                zeros.contiguous(), x.contiguous())
    _on_gpu(packed, scales, zeros, x)
    y = torch.zeros(rows, dtype=torch.float32, device=packed.device)
    with kernel_span("int4_gemv", rows=rows, cols=cols, group_size=group_size):
        _get_lib().launch_gemv_int4(
            _ptr(packed), _ptr(scales), _ptr(zeros), _ptr(x), _ptr(y),
            rows, cols, group_size, _stream())
    _check("int4_gemv")
    return y


def fp8_quantize(x, per_token: bool = True) -> Tuple:
    """
    Quantize FP32 activations to FP8 E4M3.

    :return: (quantized: int8 [rows, cols], scales: float32 [rows] or [1])

    As in the reference, per-tensor mode reads its scale from the freshly
    zeroed ``scales`` buffer, so every code saturates (reference :345-347).
    """
    import torch
    x = x.contiguous()
    _on_gpu(x)
    rows, cols = x.shape
    q = torch.zeros(rows, cols, dtype=torch.int8, device=x.device)
    n_scales = rows if per_token else 1
    scales = torch.zeros(n_scales, dtype=torch.float32, device=x.device)
    with kernel_span("fp8_quantize", rows=rows, cols=cols, per_token=per_token):
        _get_lib().launch_quantize_fp8(
            _ptr(x), _ptr(q), _ptr(scales), rows, cols, per_token, _stream())
    _check("fp8_quantize")
    return q, scales


def fp8_dequantize(q, scales, rows: int, cols: int, per_token: bool = True):
    """
    Dequantize FP8 E4M3 activations back to FP32.

    :return: torch.Tensor [rows, cols] float32 GPU
    """
    import torch
    q, scales = q.contiguous(), scales.contiguous()
    _on_gpu(q, scales)
    output = torch.zeros(rows, cols, dtype=torch.float32, device=q.device)
    _get_lib().launch_dequantize_fp8(
        _ptr(q), _ptr(scales), _ptr(output), rows, cols, per_token, _stream())
    _check("fp8_dequantize")
    return output


def speculative_verify(draft_probs, target_probs, draft_tokens, rand_vals, rand_vals2) -> Tuple:
    """Speculative-decoding verification: out of scope (stub launcher)."""
    import torch
    draft_probs, target_probs = draft_probs.contiguous(), target_probs.contiguous()
    draft_tokens, rand_vals, rand_vals2 = (draft_tokens.contiguous(), rand_vals.contiguous(),
                                           rand_vals2.contiguous())
    _on_gpu(draft_probs, target_probs, draft_tokens, rand_vals, rand_vals2)
    K, vocab = draft_probs.shape
    accepted = torch.zeros(K, dtype=torch.int32, device=draft_probs.device)
    corrected = torch.zeros(K, dtype=torch.int32, device=draft_probs.device)
    with kernel_span("speculative_verify", num_tokens=K, vocab_size=vocab):
        _get_lib().launch_verify_draft_tokens(
            _ptr(draft_probs), _ptr(target_probs), _ptr(draft_tokens), _ptr(rand_vals),
            _ptr(rand_vals2), _ptr(accepted), _ptr(corrected), K, vocab, _stream())
    _check("speculative_verify")
    return accepted, corrected


# ---------------------------------------------------------------------------
# Extensions (no reference counterpart)
# ---------------------------------------------------------------------------


def smoothquant_scale(x, smooth_scales):
    """out[r, c] = x[r, c] / smooth_scales[c] (launch_smoothquant_scale)."""
    import torch
    x, smooth_scales = x.contiguous(), smooth_scales.contiguous()
    _on_gpu(x, smooth_scales)
    rows, cols = x.shape
    out = torch.zeros(rows, cols, dtype=torch.float32, device=x.device)
    _get_lib().launch_smoothquant_scale(_ptr(x), _ptr(smooth_scales), _ptr(out), rows, cols,
                                        _stream())
    _check("smoothquant_scale")
    return out


def int4_gemv_bf16(packed, scales, zeros, x, rows: int, cols: int, group_size: int = 128):
    """y = W_int4 * x with bf16 x [cols] and bf16 y [rows], fp32 accumulation."""
    import torch
    packed, scales, zeros, x = (packed.contiguous(), scales.contiguous(),
                                zeros.contiguous(), x.contiguous())
    _on_gpu(packed, scales, zeros, x)
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
    """Runs int4_gemv_bf16 for each op in order, from one call: ops is a list
    of (packed, scales, zeros, x, y, rows, cols, group_size) with bf16 x and
    y tensors already allocated; an op may take an earlier op's y (or a
    contiguous slice of it) as its x."""
    arr = (GemvOp * max(1, len(ops)))()
    for i, (packed, scales, zeros, x, y, rows, cols, gs) in enumerate(ops):
        for t in (packed, scales, zeros, x, y):
            if not t.is_contiguous():
                raise ValueError("int4_gemv_bf16_chain: tensors must be contiguous")
        _on_gpu(packed, scales, zeros, x, y)
        arr[i] = GemvOp(_ptr(packed), _ptr(scales), _ptr(zeros), _ptr(x), _ptr(y), rows, cols, gs, 0)
    with kernel_span("int4_gemv_bf16_chain", ops=len(ops)):
        st = _get_lib().kc_gemv_int4_bf16_chain(ctypes.cast(arr, ctypes.c_void_p), len(ops),
                                                _stream())
    _check("int4_gemv_bf16_chain", st)


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
    qweight, qzeros, scales = qweight.contiguous(), qzeros.contiguous(), scales.contiguous()
    _on_gpu(qweight, qzeros, scales)
    K, N = qweight.shape[0] * 8, qweight.shape[1]
    G = K // group_size
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
    qweight, qzeros, scales = qweight.contiguous(), qzeros.contiguous(), scales.contiguous()
    _on_gpu(qweight, qzeros, scales)
    K, N = qweight.shape[0], qweight.shape[1] * 8
    G = K // group_size
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
    qx, sx, qw, sw = qx.contiguous(), sx.contiguous(), qw.contiguous(), sw.contiguous()
    _on_gpu(qx, sx, qw, sw)
    M, K = qx.shape
    N = qw.shape[0]
    if qw.shape[1] != K or sx.numel() != M or sw.numel() != N:
        raise ValueError("fp8_gemm_w8a8: shapes do not match")
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
    x, g = x.contiguous(), g.contiguous()
    _on_gpu(x, g)
    D = x.shape[-1]
    rows = x.numel() // max(D, 1)
    if g.numel() != D or g.dtype != x.dtype:
        raise ValueError("rmsnorm: g must hold D values of x's dtype")
    y = torch.empty_like(x)
    with kernel_span("rmsnorm", rows=rows, d=D):
        if x.dtype == torch.float32:
            _get_lib().launch_rmsnorm(_ptr(x), _ptr(g), _ptr(y), rows, D, eps, _stream())
            st = None
        elif x.dtype == torch.bfloat16:
            st = _get_lib().kc_rmsnorm_bf16(_ptr(x), _ptr(g), _ptr(y), rows, D, eps, _stream())
        else:
            raise TypeError("rmsnorm: float32 or bfloat16 tensors")
    _check("rmsnorm", st)
    return y


def rmsnorm_int4_gemv_bf16(h, gamma, packed, scales, zeros, rows: int, cols: int,
                           group_size: int = 128, eps: float = 1e-6):
    """y = W_int4 * bf16(rmsnorm(h) * gamma) in one launch: bf16 h, gamma
    [cols], bf16 y [rows] (kc_rmsnorm_gemv_int4_bf16)."""
    import torch
    h, gamma, packed, scales, zeros = (h.contiguous(), gamma.contiguous(), packed.contiguous(),
                                       scales.contiguous(), zeros.contiguous())
    _on_gpu(h, gamma, packed, scales, zeros)
    y = torch.empty(rows, dtype=torch.bfloat16, device=packed.device)
    with kernel_span("rmsnorm_int4_gemv_bf16", rows=rows, cols=cols, group_size=group_size):
        st = _get_lib().kc_rmsnorm_gemv_int4_bf16(_ptr(h), _ptr(gamma), eps, _ptr(packed),
                                                  _ptr(scales), _ptr(zeros), _ptr(y), rows, cols,
                                                  group_size, _stream())
    _check("rmsnorm_int4_gemv_bf16", st)
    return y


def int4_gemm_bf16(packed, scales, zeros, x, rows: int, cols: int, group_size: int = 128):
    """Y = X W^T for X bf16 [m, cols] (m <= 64) on matrix cores; Y bf16 [m, rows]."""
    import torch
    packed, scales, zeros, x = (packed.contiguous(), scales.contiguous(),
                                zeros.contiguous(), x.contiguous())
    _on_gpu(packed, scales, zeros, x)
    m = x.shape[0]
    y = torch.empty(m, rows, dtype=torch.bfloat16, device=packed.device)
    with kernel_span("int4_gemm_bf16", m=m, rows=rows, cols=cols, group_size=group_size):
        st = _get_lib().kc_gemm_int4_bf16(_ptr(packed), _ptr(scales), _ptr(zeros), _ptr(x),
                                          _ptr(y), m, rows, cols, group_size, _stream())
    _check("int4_gemm_bf16", st)
    return y


def fp8_quantize_rows(x) -> Tuple:
    """Per-row FP8 quantization of a bf16 or fp32 [rows, cols] tensor: per
    token for activations, per output channel for a weight matrix."""
    import torch
    x = x.contiguous()
    _on_gpu(x)
    rows, cols = x.shape
    q = torch.empty(rows, cols, dtype=torch.int8, device=x.device)
    s = torch.empty(rows, dtype=torch.float32, device=x.device)
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
    x = x.contiguous()
    _on_gpu(x)
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
    amax_x, amax_w = amax_x.contiguous(), amax_w.contiguous()
    _on_gpu(amax_x, amax_w)
    s = torch.empty_like(amax_x)
    st = _get_lib().kc_smooth_factors(_ptr(amax_x), _ptr(amax_w), _ptr(s), amax_x.numel(),
                                      _stream())
    _check("smooth_factors", st)
    return s


def fp8_quantize_smooth(x, smooth, mode: str = "div") -> Tuple:
    """Fused SmoothQuant + per-row FP8: ``div`` quantizes x / s (activations),
    ``mul`` quantizes x * s (weights, bf16 only)."""
    import torch
    x, smooth = x.contiguous(), smooth.contiguous()
    _on_gpu(x, smooth)
    rows, cols = x.shape
    q = torch.empty(rows, cols, dtype=torch.int8, device=x.device)
    s = torch.empty(rows, dtype=torch.float32, device=x.device)
    lib = _get_lib()
    if mode == "div":
        fn = lib.kc_quantize_fp8_smooth_div_bf16 if x.dtype == torch.bfloat16 \
            else lib.kc_quantize_fp8_smooth_div_f32
    elif mode == "mul":
        if x.dtype != torch.bfloat16:
            raise ValueError("mode='mul' takes a bf16 weight matrix")
        fn = lib.kc_quantize_fp8_smooth_mul_bf16
    else:
        raise ValueError(f"mode must be 'div' or 'mul', not {mode!r}")
    with kernel_span("fp8_quantize_smooth", rows=rows, cols=cols, mode=mode):
        st = fn(_ptr(x), _ptr(smooth), _ptr(q), _ptr(s), rows, cols, _stream())
    _check("fp8_quantize_smooth", st)
    return q, s


# ---------------------------------------------------------------------------
# torch.library registration (reference :428-479)
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
    """Register kernel_craft ops in the torch.ops namespace."""
    import torch

    lib = torch.library.Library("kernel_craft", "DEF")
    for schema in SCHEMAS.values():
        lib.define(schema)
    impl = torch.library.Library("kernel_craft", "IMPL")
    fns = {
        "flash_attention": flash_attention,
        "paged_attention": paged_attention,
        "int4_dequantize": int4_dequantize,
        "int4_gemv": int4_gemv,
        "fp8_quantize": fp8_quantize,
        "fp8_dequantize": fp8_dequantize,
        "speculative_verify": speculative_verify,
    }
    # Registered for both keys as in the reference; CPU tensors are rejected
    # by _on_gpu inside each op.
    for device in ("CPU", "CUDA"):
        for name, fn in fns.items():
            impl.impl(name, fn, device)
    globals()["_torch_lib_def"] = lib
    globals()["_torch_lib_impl"] = impl


try:
    import torch  # noqa: F401
    _register_torch_library()
    TORCH_OPS_REGISTERED = True
except Exception:
    TORCH_OPS_REGISTERED = False
