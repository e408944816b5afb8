"""Weight-only int8 / int4 quantisation — drop-in for QuantaWeave's quantization.py.

Mirrors ``QuantizedLinear`` and ``quantize_model`` (src/quantization.py:21-102):
same constructor arguments, the same registered buffers ``qweight`` /
``scales`` with byte-identical layout, the same errors.  Quantisation,
dequantisation and the forward product run as HIP kernels on the GPU; a layer
held on the CPU is processed on the current ROCm device and its buffers are
copied back.  There is no CPU implementation: without a ROCm device these
calls raise RuntimeError.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor, nn

from . import _hip, _lib


def _gpu() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("QuantizedLinear needs a ROCm device for its HIP kernels")
    return torch.device("cuda", torch.cuda.current_device())


class QuantizedLinear(nn.Module):
    """Linear layer with symmetric per-group quantised weights (src/quantization.py:21-75).

    bits=8: int8, one scale per output row (or per ``group_size`` columns if given).
    bits=4: two 4-bit values packed per byte (even column in the low nibble,
    stored as q + 8), one scale per ``group_size`` columns (default 32).
    """

    def __init__(self, in_features: int, out_features: int, bits: int = 8, group_size: Optional[int] = None) -> None:
        super().__init__()
        if bits not in (4, 8):
            raise ValueError("bits must be 4 or 8")
        group_size = group_size or (in_features if bits == 8 else 32)
        if bits == 4 and group_size % 2:
            raise ValueError("group_size must be even for 4-bit weights")
        self.in_features, self.out_features, self.bits, self.group_size = in_features, out_features, bits, group_size
        self.padded = -(-in_features // group_size) * group_size
        groups = self.padded // group_size
        stored = self.padded if bits == 8 else self.padded // 2
        self.register_buffer("qweight", torch.zeros(out_features, stored, dtype=torch.int8 if bits == 8 else torch.uint8))
        self.register_buffer("scales", torch.ones(out_features, groups))

    @property
    def w_format(self) -> int:
        return _lib.QW_I8 if self.bits == 8 else _lib.QW_U4

    @classmethod
    def from_linear(cls, linear: nn.Linear, bits: int = 8, group_size: Optional[int] = None) -> "QuantizedLinear":
        if linear.bias is not None:
            raise ValueError("bias is not supported")
        layer = cls(linear.in_features, linear.out_features, bits, group_size).to(linear.weight.device)
        weight = linear.weight.detach()
        if weight.dtype not in _hip.FLOAT_DTYPES:
            weight = weight.float()
        dev = weight.device if weight.device.type == "cuda" else _gpu()
        w = weight.to(dev).contiguous()
        q = torch.empty(layer.qweight.shape, dtype=layer.qweight.dtype, device=dev)
        s = torch.empty(layer.scales.shape, dtype=torch.float32, device=dev)
        _lib.call("qw_quantize", _hip.ptr(w), _hip.act_code(w, "quantize"), layer.out_features, layer.in_features,
                  bits, layer.group_size, _hip.ptr(q), _hip.ptr(s), _hip.stream(dev))
        layer.qweight.copy_(q)
        layer.scales.copy_(s)
        return layer

    def dequantize(self) -> Tensor:
        """fp32 [out, in] = q * scale per group (src/quantization.py:61-69)."""
        dev = self.qweight.device if self.qweight.device.type == "cuda" else _gpu()
        q = self.qweight.to(dev).contiguous()
        s = self.scales.to(dev, torch.float32).contiguous()
        out = torch.empty(self.out_features, self.in_features, dtype=torch.float32, device=dev)
        _lib.call("qw_dequantize", _hip.ptr(q), _hip.ptr(s), self.bits, self.out_features, self.in_features,
                  self.group_size, _hip.ptr(out), _hip.stream(dev))
        return out.to(self.qweight.device)

    def forward(self, x: Tensor) -> Tensor:
        """F.linear(x, dequantize().to(x.dtype)) (src/quantization.py:71-72) with the
        dequantisation done in registers of the HIP kernel."""
        _hip.require_device(x, "QuantizedLinear.forward")
        act = _hip.act_code(x, "QuantizedLinear.forward")
        lead = x.shape[:-1]
        flat = x.reshape(-1, self.in_features).contiguous()
        rows = flat.size(0)
        out = torch.empty(rows, self.out_features, dtype=x.dtype, device=x.device)
        if rows:
            offsets = torch.tensor([0, rows], dtype=torch.int32, device=x.device)
            scales = self.scales if self.scales.dtype == torch.float32 else self.scales.float()
            _lib.call("qw_grouped_matmul", _hip.ptr(flat), act, _hip.ptr(self.qweight), self.w_format,
                      _hip.ptr(scales.contiguous()), self.group_size, 1, self.out_features, self.in_features,
                      _hip.ptr(offsets), rows, 0, _hip.ptr(out), _hip.stream(x.device))
        return out.reshape(*lead, self.out_features)

    def stored_bytes(self) -> int:
        return self.qweight.numel() * self.qweight.element_size() + self.scales.numel() * self.scales.element_size()

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, bits={self.bits}, group_size={self.group_size}"


def quantize_model(model: nn.Module, bits: int = 8, group_size: Optional[int] = None, quantize_lm_head: bool = False) -> dict:
    """Replace expert weights (and optionally lm_head) in place; returns size statistics
    (src/quantization.py:78-102).  Works on any module whose MoE layers expose
    ``.experts`` of gate/up/down projections: ``model.blocks[i].moe`` as in the
    reference model, or TopKMoE modules anywhere in the tree."""
    if getattr(model, "expert_parallel", None) is not None:
        raise ValueError("consolidate an expert-parallel model before quantizing it")
    before = after = replaced = 0

    def swap(parent: nn.Module, name: str) -> None:
        nonlocal before, after, replaced
        linear = getattr(parent, name)
        if isinstance(linear, QuantizedLinear):
            raise ValueError("model is already quantized")
        quantized = QuantizedLinear.from_linear(linear, bits, group_size)
        before += linear.weight.numel() * linear.weight.element_size()
        after += quantized.stored_bytes()
        replaced += 1
        setattr(parent, name, quantized)

    from .moe import TopKMoE

    if hasattr(model, "blocks"):
        moes = [block.moe for block in model.blocks]
    else:
        moes = [m for m in model.modules() if isinstance(m, TopKMoE)]
    for moe in moes:
        for expert in moe.experts:
            for name in ("gate", "up", "down"):
                swap(expert, name)
    if quantize_lm_head:
        swap(model, "lm_head")
    return {"bits": bits, "group_size": group_size, "replaced_layers": replaced, "bytes_before": before,
            "bytes_after": after, "compression": before / after if after else None}
