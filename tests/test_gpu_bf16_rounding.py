"""fp32 -> bf16 rounding of the kernels, bit for bit.

Every bf16 store of the library (expert outputs, hidden rows, combine sums)
goes through one rounding: round to nearest, ties to even, on the fp32 bits,
(bits + 0x7fff + lsb) >> 16, a NaN keeping its sign and top payload with the
quiet bit set.  A combine with one route per token and weight 1 from fp32
rows into a bf16 output rounds y * 1 and then 0 + that (which only turns -0
into +0), so it checks the rounding on arbitrary bit patterns: ties, the
largest finite values, infinities, denormals and quiet NaNs.
"""

import numpy as np
import pytest
import torch

from quantaweave_amd import _hip, _lib
from quantaweave_amd._lib import QW_BF16, QW_F32


def rne_bf16_bits(f32: np.ndarray) -> np.ndarray:
    """The rounding restated on the CPU (uint16 bits of the bf16 values)."""
    u = f32.view(np.uint32).astype(np.uint64)
    rne = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    nan = ((u >> 16) | 0x40) & 0xFFFF
    return np.where((u & 0x7FFFFFFF) > 0x7F800000, nan, rne).astype(np.uint16)


def test_rne_restatement_known_answers():
    """The CPU restatement against values whose bf16 rounding is known."""
    f = np.array([1.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 1.0 + 2.0 ** -8 + 2.0 ** -20, -2.5, 65504.0,
                  3.3895313892515355e38, np.inf, -np.inf], dtype=np.float32)
    want = np.array([0x3F80, 0x3F80, 0x3F82, 0x3F81, 0xC020, 0x4780, 0x7F7F, 0x7F80, 0xFF80], dtype=np.uint16)
    assert np.array_equal(rne_bf16_bits(f), want)
    # torch's own conversion agrees on every non-NaN value
    r = np.random.default_rng(0).integers(0, 2 ** 32, 100000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    r = r[~np.isnan(r)]
    got = torch.from_numpy(r.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(rne_bf16_bits(r), got)


@pytest.mark.gpu
def test_kernel_rounding_is_rne_bit_for_bit():
    print("case bf16 rounding through qw_moe_combine_weighted", flush=True)
    rng = np.random.default_rng(1)
    edges = []
    for sign in (0, 1):
        for e in range(256):
            for m in (0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x10000, 0x17FFF, 0x18000, 0x18001, 0x7F7FFF, 0x7F8000,
                      0x7FFFFF, 0x400000):
                edges.append((sign << 31) | (e << 23) | m)
    bits = np.concatenate([np.array(edges, dtype=np.uint32),
                           rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32)])
    # quiet NaNs only: how an add treats a signalling NaN is not what this checks
    snan = ((bits & 0x7F800000) == 0x7F800000) & ((bits & 0x7FFFFF) != 0) & ((bits & 0x400000) == 0)
    bits = bits[~snan]
    T, D = 1024, len(bits) // 1024 // 8 * 8  # rows of 8-value vectors, the combine's vector path
    y = bits[: T * D].view(np.float32).reshape(T, D)
    # the combine rounds the route's term, then the sum 0 + term (-0 becomes +0)
    term = (rne_bf16_bits(y * np.float32(1)).astype(np.uint32) << 16).view(np.float32)
    expect = rne_bf16_bits(np.float32(0) + term)
    dev = torch.device("cuda")
    yd = torch.from_numpy(y.copy()).to(dev)
    slot = torch.arange(T, dtype=torch.int32, device=dev)
    idx = torch.zeros(T, dtype=torch.int32, device=dev)
    w = torch.ones(T, dtype=torch.float32, device=dev)
    out = torch.empty(T, D, dtype=torch.bfloat16, device=dev)
    _lib.call("qw_moe_combine_weighted", _hip.ptr(yd), QW_F32, _hip.ptr(slot), _hip.ptr(idx), _hip.ptr(w), T, 1, D,
              _hip.ptr(out), QW_BF16, _hip.stream(dev))
    torch.cuda.synchronize()
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)
    bad = np.flatnonzero(got.ravel() != expect.ravel())
    assert bad.size == 0, [(hex(int(y.ravel().view(np.uint32)[i])), hex(int(got.ravel()[i])),
                            hex(int(expect.ravel()[i]))) for i in bad[:8]]
