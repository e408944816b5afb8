"""ctypes binding of ``libqwmoe.so`` (the C ABI declared in include/qwmoe.h).

The library is loaded from this package directory only; there is no other
implementation to fall back to, so a missing library is an ImportError-like
RuntimeError at first use.  Status codes map to the reference's exception
types: QW_ERR_INVALID -> ValueError, everything else -> RuntimeError.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libqwmoe.so"

QW_F32, QW_BF16, QW_I8, QW_U4, QW_BF16T, QW_F16, QW_F16T = 0, 1, 2, 3, 4, 5, 6
QW_OK, QW_ERR_INVALID, QW_ERR_UNSUPPORTED, QW_ERR_HIP, QW_ERR_WORKSPACE = 0, -1, -2, -3, -4
QW_PATH_AUTO, QW_PATH_GENERAL, QW_PATH_MFMA, QW_PATH_STREAM = 0, 1, 2, 3

P = ctypes.c_void_p
I32, I64, F32, F64, SZ = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_double, ctypes.c_size_t

# name -> (restype, argtypes); kept in the order of include/qwmoe.h
SIGNATURES = {
    "qw_last_error": (ctypes.c_char_p, []),
    "qw_abi_version": (I32, []),
    "qw_moe_capacity": (I64, [I64, I64, I64, F64, F64, I64, I32]),
    "qw_moe_route_workspace_bytes": (SZ, [I64, I64, I64]),
    "qw_moe_route": (I32, [P, I32, I64, P, I32, I64, I64, I64, I64, F32, P, P, P, P, P, P, SZ, P]),
    "qw_moe_route_from_logits": (I32, [P, I64, I64, I64, P, P, P, P, P]),
    "qw_moe_plan_workspace_bytes": (SZ, [I64, I64, I64]),
    "qw_moe_plan": (I32, [P, P, I64, I64, I64, I64, P, P, P, P, P, P, P, P, P, P, SZ, P]),
    "qw_moe_permute": (I32, [P, I32, I64, P, P, I64, P, P]),
    "qw_moe_experts_workspace_bytes": (SZ, [I64, I64, I64, I64, I32]),
    "qw_moe_experts": (I32, [P, I32, P, P, I64, I64, I64, I64, I64, I32, I64, I64, P, P, P, P, P, P, P, P, P, SZ, P]),
    "qw_moe_experts_on_path": (I32, [I32, P, I32, P, P, I64, I64, I64, I64, I64, I32, I64, I64, P, P, P, P, P, P,
                                     P, P, P, SZ, P]),
    "qw_moe_combine": (I32, [P, I32, P, P, I64, I64, I64, P, P]),
    "qw_moe_balance": (I32, [P, P, I64, I64, I64, P, P, P]),
    "qw_moe_balance_workspace_bytes": (SZ, [I64, I64]),
    "qw_moe_balance_ws": (I32, [P, P, I64, I64, I64, P, P, P, SZ, P]),
    "qw_moe_forward_workspace_bytes": (SZ, [I64, I64, I64, I64, I64, I32]),
    "qw_moe_forward": (I32, [P, I32, I64, I64, P, I32, F32, P, I64, I64, I64, I64, I32, I64, I64,
                             P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, SZ, P]),
    "qw_moe_decode_step_workspace_bytes": (SZ, [I64, I64, I64, I64, I64, I32]),
    "qw_moe_decode_step": (I32, [P, P, I64, I64, P, F32, P, I64, I64, I64, I32, I32, I64, I64,
                                 P, P, P, P, P, P, P, P, P, P, P, SZ, P]),
    "qw_init": (I32, []),
    "qw_moe_decode_step_noalloc_scratch_bytes": (SZ, []),
    "qw_moe_decode_step_noalloc": (I32, [P, P, I64, I64, P, F32, P, I64, I64, I64, I32, I32, I64, I64,
                                         P, P, P, P, P, P, P, P, P, P, P]),
    "qw_quantize": (I32, [P, I32, I64, I64, I32, I64, P, P, P]),
    "qw_dequantize": (I32, [P, P, I32, I64, I64, I64, P, P]),
    "qw_pack_bf16_tiles": (I32, [P, I64, I64, I64, P, P]),
    "qw_grouped_matmul": (I32, [P, I32, P, I32, P, I64, I64, I64, I64, P, I64, I64, P, P]),
    "qw_moe_combine_static": (I32, [P, I32, P, P, P, I64, I64, I64, P, I32, P]),
    "qw_grouped_matmul_backward_workspace_bytes": (SZ, [I64, I64, I64, I64, I32]),
    "qw_grouped_matmul_backward": (I32, [P, P, P, I32, I64, I64, I64, P, I64, I64, P, I32, P, I32, P, SZ, P]),
    "qw_moe_experts_save": (I32, [P, I32, P, P, I64, I64, I64, I64, I64, I32, I64, I64, P, P, P, P, P, P, P, P,
                                  P, P, P, P, P, SZ, P]),
    "qw_swiglu": (I32, [P, P, I32, I64, P, P]),
    "qw_swiglu_backward": (I32, [P, P, P, I32, I64, P, P, P]),
    "qw_moe_combine_weighted": (I32, [P, I32, P, P, P, I64, I64, I64, P, I32, P]),
    "qw_moe_combine_backward": (I32, [P, I32, P, I32, P, P, I64, I64, I64, P, P, P]),
    "qw_moe_route_backward": (I32, [P, P, P, P, P, P, P, I64, I64, I64, F32, P, P]),
}

_lib: ctypes.CDLL | None = None


class QWError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load libqwmoe.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"the HIP MoE library {LIB_PATH} is not built; run `python -m quantaweave_amd.build`")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status == QW_OK:
        return
    msg = load().qw_last_error().decode(errors="replace")
    text = f"{what}: {msg}" if msg else f"{what} failed with status {status}"
    if status == QW_ERR_INVALID:
        raise ValueError(text)
    raise RuntimeError(text)


def call(name: str, *args) -> int:
    """Call an entry point that returns a status; raise on failure."""
    status = getattr(load(), name)(*args)
    check(status, name)
    return status


def available() -> bool:
    return LIB_PATH.exists()
