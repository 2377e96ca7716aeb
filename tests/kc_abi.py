"""Direct C-ABI access for tests: the library as the reference's ctypes
bridge loads it, plus the list of symbols include/kernel_craft.h declares."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "kernel_craft.h"


def lib() -> ctypes.CDLL:
    import kernel_craft_torch_ops as ops
    return ops._get_lib()


def header_functions() -> list[str]:
    """Every function name declared in include/kernel_craft.h."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\(", text)
    skip = {"if", "defined", "sizeof"}
    return sorted({n for n in names if n not in skip and (
        n.startswith("launch_") or n.startswith("kc_") or n.startswith("nccl_"))})


def ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def stream() -> ctypes.c_void_p:
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def check(name: str, status: int | None = None) -> None:
    L = lib()
    code = L.kc_get_last_error()
    if status:
        code = status
    if code:
        raise RuntimeError(f"{name}: kc_status {code}: {L.kc_last_error_string().decode()}")
