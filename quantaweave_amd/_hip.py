"""Tensor plumbing for the C ABI: device checks, pointers, dtype codes, stream."""

from __future__ import annotations

import torch

from . import _lib

_ACT = {torch.float32: _lib.QW_F32, torch.bfloat16: _lib.QW_BF16, torch.float16: _lib.QW_F16}
# 16-bit float types and the codes of their plain and tiled weight formats
HALF = {torch.bfloat16: (_lib.QW_BF16, _lib.QW_BF16T), torch.float16: (_lib.QW_F16, _lib.QW_F16T)}
FLOAT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def require_device(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda" or not torch.cuda.is_available():
        raise RuntimeError(f"{what}: the HIP MoE kernels need a ROCm (cuda) device tensor, got {t.device}")


def act_code(t: torch.Tensor, what: str) -> int:
    try:
        return _ACT[t.dtype]
    except KeyError:
        raise ValueError(f"{what}: dtype {t.dtype} is not supported (float32, bfloat16 or float16)") from None


def ptr(t: torch.Tensor | None) -> int | None:
    """Device address of a tensor for a `void*` argument (ctypes converts the
    int; None is NULL)."""
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    """The current HIP stream of `device`, for a `void* stream` argument."""
    return torch.cuda.current_stream(device).cuda_stream


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
