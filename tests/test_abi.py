"""The C ABI library loads and exports every symbol include/qwmoe.h declares.

Only host-side behaviour is exercised here (argument validation, the capacity
arithmetic): nothing in this file launches a kernel."""

import ctypes
import re
from pathlib import Path

import pytest

import oracle
from quantaweave_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "qwmoe.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qw_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    names = declared_symbols()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), "python binding and header disagree"


def test_abi_version_and_empty_error():
    lib = _lib.load()
    assert lib.qw_abi_version() == 1
    assert isinstance(lib.qw_last_error(), bytes)


@pytest.mark.parametrize("T,k,E,cf,scale,minc,drop", [
    (512, 2, 8, 1.25, 1.0, 4, 1), (8192, 2, 64, 1.25, 1.0, 4, 1), (64, 2, 64, 0.0, 1.0, 4, 1),
    (16, 2, 64, 0.0, 1.0, 4, 1), (4096, 2, 64, 1.0, 1.0, 4, 1), (100, 2, 8, 1.25, 0.5, 4, 1),
    (100, 2, 8, 1.25, 1.0, 4, 0), (3, 1, 8, 0.1, 1.0, 4, 1), (24, 2, 6, 0.6, 1.0, 2, 1), (7, 3, 5, 0.7, 1.3, 1, 1),
])
def test_capacity_entry_point_matches_oracle(T, k, E, cf, scale, minc, drop):
    got = _lib.load().qw_moe_capacity(T, k, E, cf, scale, minc, drop)
    assert got == oracle.capacity(T, k, E, cf, scale, minc, bool(drop))


def test_invalid_arguments_are_reported_before_any_launch():
    lib = _lib.load()
    # experts = 0 is rejected with QW_ERR_INVALID and a message
    st = lib.qw_moe_route_from_logits(None, 4, 0, 1, None, None, None, None, None)
    assert st == _lib.QW_ERR_INVALID and b"experts" in lib.qw_last_error()
    st = lib.qw_moe_route_from_logits(None, 4, 8, 9, None, None, None, None, None)
    assert st == _lib.QW_ERR_INVALID and b"top_k" in lib.qw_last_error()
    st = lib.qw_quantize(None, 0, 4, 8, 3, 8, None, None, None)
    assert st == _lib.QW_ERR_INVALID and b"bits" in lib.qw_last_error()
    st = lib.qw_quantize(None, 0, 4, 8, 4, 7, None, None, None)
    assert st == _lib.QW_ERR_INVALID and b"even" in lib.qw_last_error()
    st = lib.qw_moe_plan(None, None, 4, 2, 8, 4, None, None, None, None, None, None, None, None, None, None, 0, None)
    assert st == _lib.QW_ERR_INVALID
    assert lib.qw_moe_capacity(4, 0, 8, 1.0, 1.0, 4, 1) < 0
    with pytest.raises(ValueError, match="top_k"):
        _lib.call("qw_moe_route_from_logits", None, 4, 8, 9, None, None, None, None, None)


def test_workspace_sizes_are_positive_and_monotone():
    lib = _lib.load()
    a = lib.qw_moe_forward_workspace_bytes(512, 256, 8, 2, 512, _lib.QW_F32)
    b = lib.qw_moe_forward_workspace_bytes(8192, 2048, 64, 2, 1024, _lib.QW_BF16)
    assert 0 < a < b
    assert lib.qw_moe_plan_workspace_bytes(8192, 2, 64) > 8192 * 2 * 8
    assert lib.qw_moe_experts_workspace_bytes(100, 8, 64, 128, _lib.QW_BF16) >= 100 * 128 * 2


def test_decode_step_validation_and_workspace():
    lib = _lib.load()
    # an unknown compute dtype (7); top_k > experts; missing workspace
    st = lib.qw_moe_decode_step(None, None, 1, 64, None, 1.0, None, 8, 2, 32, 7, _lib.QW_BF16, 0, 0,
                                None, None, None, None, None, None, None, None, None, None, None, 0, None)
    assert st == _lib.QW_ERR_INVALID and b"compute dtype" in lib.qw_last_error()
    st = lib.qw_moe_decode_step(None, None, 1, 64, None, 1.0, None, 8, 9, 32, _lib.QW_BF16, _lib.QW_BF16, 0, 0,
                                None, None, None, None, None, None, None, None, None, None, None, 0, None)
    assert st == _lib.QW_ERR_INVALID and b"top_k" in lib.qw_last_error()
    fake = ctypes.c_void_p(16)    # never dereferenced: the workspace check fails first
    st = lib.qw_moe_decode_step(fake, None, 1, 64, fake, 1.0, None, 8, 2, 32, _lib.QW_BF16, _lib.QW_BF16, 0, 0,
                                fake, None, fake, None, fake, None, fake, None, fake, fake, fake, 16, None)
    assert st == _lib.QW_ERR_WORKSPACE and b"workspace" in lib.qw_last_error()
    # zero tokens is a no-op that touches nothing
    assert lib.qw_moe_decode_step(None, None, 0, 64, None, 1.0, None, 8, 2, 32, _lib.QW_BF16, _lib.QW_BF16, 0, 0,
                                  None, None, None, None, None, None, None, None, None, None, None, 0, None) == 0
    one = lib.qw_moe_decode_step_workspace_bytes(1, 4096, 64, 2, 1408, _lib.QW_BF16)
    assert 0 < one < lib.qw_moe_decode_step_workspace_bytes(16, 4096, 64, 2, 1408, _lib.QW_BF16)
    assert lib.qw_moe_decode_step_workspace_bytes(1, 4096, 64, 2, 1408, 7) == 0


def test_backward_entry_points_validate_before_any_launch():
    lib = _lib.load()
    bad = _lib.QW_ERR_INVALID
    # grouped backward: plain fp32/bf16 only, offsets required
    assert lib.qw_grouped_matmul_backward(None, None, None, _lib.QW_I8, 8, 16, 16, None, 4, 0, None, 0, None,
                                          _lib.QW_I8, None, 0, None) == bad
    assert b"dtype" in lib.qw_last_error()
    assert lib.qw_grouped_matmul_backward(None, None, None, _lib.QW_F32, 8, 16, 16, None, 4, 0, None, 0, None,
                                          _lib.QW_F32, None, 0, None) == bad
    assert lib.qw_grouped_matmul_backward_workspace_bytes(8, 64, 64, 100, _lib.QW_BF16) > 64 * 64 * 8 * 2
    assert lib.qw_grouped_matmul_backward_workspace_bytes(0, 64, 64, 100, _lib.QW_BF16) == 0
    assert b"offsets" in lib.qw_last_error()
    assert lib.qw_swiglu(None, None, _lib.QW_F32, -1, None, None) == bad
    assert lib.qw_swiglu_backward(None, None, None, _lib.QW_U4, 8, None, None, None) == bad
    # combine and route backward: top_k <= 64
    assert lib.qw_moe_combine_backward(None, _lib.QW_F32, None, _lib.QW_F32, None, None, 4, 65, 8, None, None,
                                       None) == bad
    assert lib.qw_moe_route_backward(None, None, None, None, None, None, None, 4, 128, 65, 1.0, None, None) == bad
    assert b"top_k" in lib.qw_last_error()
    assert lib.qw_moe_route_backward(None, None, None, None, None, None, None, 4, 8, 2, 0.0, None, None) == bad
    assert lib.qw_moe_combine_weighted(None, _lib.QW_F32, None, None, None, 4, 2, 8, None, _lib.QW_I8, None) == bad
    # nothing to do is not an error
    assert lib.qw_moe_route_backward(None, None, None, None, None, None, None, 0, 8, 2, 1.0, None, None) == 0
    assert lib.qw_swiglu(None, None, _lib.QW_BF16, 0, None, None) == 0
