"""Synthetic MoE-layer workloads used by the benchmark, the smoke run and the tests.

Each workload is one MoE FFN layer: activations N(0,1), router and expert
weights N(0, 0.02), a fixed seed, generated on the device with torch's
seeded generator (no dataset, no checkpoint).  Quantised workloads quantise
fp32 expert weights with the library's own ``qw_quantize`` (the layout of
src/quantization.py:43-59).  The skewed workload adds a selection-only expert
bias (src/quantweave_moe_model.py:133-135) of -1.2*ln(rank)*0.4, whose top-1
selection histogram fits Zipf(s=1.2) best among scales 0.1..1.4 in 0.1 steps.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from . import _hip, _lib


@dataclass(frozen=True)
class Workload:
    name: str
    tokens: int
    d_model: int
    experts: int
    d_ff: int
    top_k: int
    capacity_factor: float   # 0 = no capacity drop
    act: str                 # "f32" | "bf16" | "f16"
    weights: str             # "f32" | "bf16" | "f16" | "i8" | "u4"
    seed: int
    group_size: int | None = None
    zipf: float = 0.0        # Zipf exponent of the selection bias (0 = none)
    batch: int = 1

    @property
    def seq(self) -> int:
        return self.tokens // self.batch

    def capacity(self, min_capacity: int = 4) -> int:
        if self.capacity_factor > 0:
            return max(min_capacity, math.ceil(self.tokens * self.top_k / self.experts * self.capacity_factor))
        return self.tokens * self.top_k


WORKLOADS = {
    w.name: w for w in [
        Workload("fp32-plumbing-T512-d256-E8-f512-k2", 512, 256, 8, 512, 2, 1.25, "f32", "f32", 1001, batch=4),
        Workload("bf16-prefill-T8192-d2048-E64-f1024-k2", 8192, 2048, 64, 1024, 2, 1.25, "bf16", "bf16", 1002, batch=8),
        Workload("int8-decode-T64-d2048-E64-f1024-k2", 64, 2048, 64, 1024, 2, 0.0, "bf16", "i8", 1003, batch=64),
        Workload("int4-decode-T16-d4096-E64-f1408-k2", 16, 4096, 64, 1408, 2, 0.0, "bf16", "u4", 1004, group_size=32,
                 batch=16),
        Workload("skewed-T4096-d2048-E64-f1024-k2", 4096, 2048, 64, 1024, 2, 1.0, "bf16", "bf16", 1005, zipf=1.2),
        # the prefill layer with weight-only quantised experts (int8 per output
        # row, int4 in groups of 32): the matrix-core path with in-register dequant
        Workload("int8-prefill-T8192-d2048-E64-f1024-k2", 8192, 2048, 64, 1024, 2, 1.25, "bf16", "i8", 1006, batch=8),
        Workload("int4-prefill-T8192-d2048-E64-f1024-k2", 8192, 2048, 64, 1024, 2, 1.25, "bf16", "u4", 1007,
                 group_size=32, batch=8),
        # the prefill layer in fp16 (the reference's fp16 precision): fp16 matrix cores
        Workload("f16-prefill-T8192-d2048-E64-f1024-k2", 8192, 2048, 64, 1024, 2, 1.25, "f16", "f16", 1008, batch=8),
    ]
}

HEADLINE = "bf16-prefill-T8192-d2048-E64-f1024-k2"
ZIPF_BETA = 0.4

_TORCH = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
_CODE = {"f32": _lib.QW_F32, "bf16": _lib.QW_BF16, "f16": _lib.QW_F16}


def scaled(w: Workload, tokens: int | None = None, d_model: int | None = None, experts: int | None = None,
           d_ff: int | None = None) -> Workload:
    """A smaller copy of a workload for oracle-sized parity runs."""
    return Workload(f"{w.name}@small", tokens or w.tokens, d_model or w.d_model, experts or w.experts, d_ff or w.d_ff,
                    w.top_k, w.capacity_factor, w.act, w.weights, w.seed, w.group_size, w.zipf, 1)


@dataclass
class Layer:
    """Device tensors of one synthetic MoE layer."""

    w: Workload
    x: torch.Tensor                  # [T, d] act dtype
    router: torch.Tensor             # [E, d] act dtype (the module dtype)
    fmt: int
    gate: torch.Tensor
    up: torch.Tensor
    down: torch.Tensor
    gate_s: torch.Tensor | None = None
    up_s: torch.Tensor | None = None
    down_s: torch.Tensor | None = None
    group_in: int = 0
    group_ff: int = 0
    bias: torch.Tensor | None = None
    extra: dict = field(default_factory=dict)

    def weight_args(self) -> list:
        """Weight arguments of the C ABI; 16-bit layers pass their QW_BF16T / QW_F16T tiles when they have them."""
        if "tiles" in self.extra:
            g, u, d = self.extra["tiles"]
            code = _lib.QW_BF16T if self.fmt == _lib.QW_BF16 else _lib.QW_F16T
            return [code, 0, 0, _hip.ptr(g), None, _hip.ptr(u), None, _hip.ptr(d), None]
        return [self.fmt, self.group_in, self.group_ff, _hip.ptr(self.gate), _hip.ptr(self.gate_s),
                _hip.ptr(self.up), _hip.ptr(self.up_s), _hip.ptr(self.down), _hip.ptr(self.down_s)]

    def add_tiles(self) -> "Layer":
        """Pack 16-bit weights into QW_BF16T / QW_F16T tiles (as the TopKMoE module does) and use them."""
        from .moe import can_tile, tile_bf16
        if self.fmt in (_lib.QW_BF16, _lib.QW_F16) and all(can_tile(t) for t in (self.gate, self.up, self.down)):
            self.extra["tiles"] = (tile_bf16(self.gate), tile_bf16(self.up), tile_bf16(self.down))
        return self

    def expert_bytes(self) -> int:
        """Stored bytes of one expert's three projections (weights + scales)."""
        n = 0
        for t in (self.gate, self.up, self.down, self.gate_s, self.up_s, self.down_s):
            if t is not None:
                n += t[0].numel() * t.element_size()
        return n


def _quantize_stack(w32: torch.Tensor, bits: int, group: int) -> tuple[torch.Tensor, torch.Tensor]:
    E, rows, cols = w32.shape
    padded = -(-cols // group) * group
    stored = padded if bits == 8 else padded // 2
    q = torch.empty(E, rows, stored, dtype=torch.int8 if bits == 8 else torch.uint8, device=w32.device)
    s = torch.empty(E, rows, padded // group, dtype=torch.float32, device=w32.device)
    dev = w32.device
    for e in range(E):
        _lib.call("qw_quantize", _hip.ptr(w32[e]), _lib.QW_F32, rows, cols, bits, group, _hip.ptr(q[e]),
                  _hip.ptr(s[e]), _hip.stream(dev))
    return q, s


def zipf_bias(experts: int, exponent: float = 1.2, beta: float = ZIPF_BETA) -> torch.Tensor:
    ranks = torch.arange(1, experts + 1, dtype=torch.float64)
    return (-exponent * torch.log(ranks) * beta).float()


def build_layer(w: Workload, device: torch.device | str = "cuda") -> Layer:
    device = torch.device(device)
    g = torch.Generator(device=device)
    g.manual_seed(w.seed)
    act = _TORCH[w.act]
    x = torch.randn(w.tokens, w.d_model, generator=g, device=device).to(act)
    router = (torch.randn(w.experts, w.d_model, generator=g, device=device) * 0.02).to(act)

    def normal(*shape):
        return torch.randn(*shape, generator=g, device=device) * 0.02

    gate32 = normal(w.experts, w.d_ff, w.d_model)
    up32 = normal(w.experts, w.d_ff, w.d_model)
    down32 = normal(w.experts, w.d_model, w.d_ff)
    layer: Layer
    if w.weights in _TORCH:
        wt = _TORCH[w.weights]
        layer = Layer(w, x, router, _CODE[w.weights], gate32.to(wt).contiguous(), up32.to(wt).contiguous(),
                      down32.to(wt).contiguous())
    else:
        bits = 8 if w.weights == "i8" else 4
        g_in = w.group_size or (w.d_model if bits == 8 else 32)
        g_ff = w.group_size or (w.d_ff if bits == 8 else 32)
        gq, gs = _quantize_stack(gate32, bits, g_in)
        uq, us = _quantize_stack(up32, bits, g_in)
        dq, ds = _quantize_stack(down32, bits, g_ff)
        layer = Layer(w, x, router, _lib.QW_I8 if bits == 8 else _lib.QW_U4, gq, uq, dq, gs, us, ds, g_in, g_ff)
    del gate32, up32, down32
    if w.zipf:
        layer.bias = zipf_bias(w.experts, w.zipf).to(device)
    return layer


class LayerRunner:
    """Preallocated outputs + workspace for repeated qw_moe_forward calls on one layer."""

    def __init__(self, layer: Layer, capacity: int | None = None) -> None:
        w = layer.w
        dev = layer.x.device
        self.layer = layer
        self.capacity = w.capacity() if capacity is None else capacity
        T, E, K = w.tokens, w.experts, w.top_k
        R = T * K
        self.act = _CODE[w.act]
        self.out = torch.empty_like(layer.x)
        self.probs = torch.empty(T, E, dtype=torch.float32, device=dev)
        self.top_idx = torch.empty(T, K, dtype=torch.int32, device=dev)
        self.top_w = torch.empty(T, K, dtype=torch.float32, device=dev)
        self.counts = torch.empty(E, dtype=torch.int32, device=dev)
        self.kept_counts = torch.empty(E, dtype=torch.int32, device=dev)
        self.totals = torch.zeros(2, dtype=torch.int32, device=dev)
        self.dropped_token = torch.empty(R, dtype=torch.int32, device=dev)
        self.dropped_expert = torch.empty(R, dtype=torch.int32, device=dev)
        self.ws_bytes = _lib.load().qw_moe_forward_workspace_bytes(T, w.d_model, E, K, w.d_ff, self.act)
        self.ws = _hip.workspace(self.ws_bytes, dev)
        self.stream = _hip.stream(dev)
        lay = layer
        self._args = [
            _hip.ptr(lay.x), self.act, T, w.d_model, _hip.ptr(lay.router), self.act, 1.0, _hip.ptr(lay.bias), E, K,
            self.capacity, w.d_ff, *lay.weight_args(), _hip.ptr(self.out), _hip.ptr(self.probs),
            _hip.ptr(self.top_idx), _hip.ptr(self.top_w), _hip.ptr(self.counts), _hip.ptr(self.kept_counts),
            _hip.ptr(self.totals), _hip.ptr(self.dropped_token), _hip.ptr(self.dropped_expert), _hip.ptr(self.ws),
            self.ws_bytes, self.stream,
        ]
        self._fn = _lib.load().qw_moe_forward

    def __call__(self) -> None:
        st = self._fn(*self._args)
        if st:
            _lib.check(st, "qw_moe_forward")

    def workspace_view(self, name: str) -> torch.Tensor:
        """Views of the forward workspace (layout of forward_workspace_bytes in qw_api.hip)."""
        w = self.layer.w
        T, E, K, D = w.tokens, w.experts, w.top_k, w.d_model
        R = T * K
        off = 0

        def take(nbytes):
            nonlocal off
            off = (off + 255) // 256 * 256
            start = off
            off += nbytes
            return start

        logits = take(T * E * 4)
        slot_token = take(R * 4)
        slot_weight = take(R * 4)
        route_slot = take(R * 4)
        kept_offsets = take((E + 1) * 4)
        y = take(R * D * (4 if self.act == _lib.QW_F32 else 2))
        views = {
            "logits": (logits, torch.float32, (T, E)),
            "slot_token": (slot_token, torch.int32, (R,)),
            "slot_weight": (slot_weight, torch.float32, (R,)),
            "route_slot": (route_slot, torch.int32, (R,)),
            "kept_offsets": (kept_offsets, torch.int32, (E + 1,)),
            "y": (y, _TORCH[w.act], (R, D)),
        }
        start, dt, shape = views[name]
        n = 1
        for s in shape:
            n *= s
        nbytes = n * torch.empty((), dtype=dt).element_size()
        return self.ws[start:start + nbytes].view(dt).view(*shape)


class DecodeRunner:
    """Preallocated buffers for repeated qw_moe_decode_step calls on one layer:
    `tokens` rows of fp32 normed input, the fp32 router (the layer's router
    widened), the layer's experts in their stored format, compute in the
    layer's activation dtype (bf16 or fp16)."""

    def __init__(self, layer: Layer, tokens: int = 1, seed: int = 0) -> None:
        w = layer.w
        dev = layer.x.device
        self.layer = layer
        self.tokens = tokens
        T, E, K = tokens, w.experts, w.top_k
        g = torch.Generator(device=dev)
        g.manual_seed(w.seed + 100 + seed)
        self.x = torch.randn(T, w.d_model, generator=g, device=dev)
        self.residual = torch.randn(T, w.d_model, generator=g, device=dev)
        self.router = layer.router.float().contiguous()
        self.out = torch.empty(T, w.d_model, dtype=torch.float32, device=dev)
        self.probs = torch.empty(T, E, dtype=torch.float32, device=dev)
        self.top_idx = torch.empty(T, K, dtype=torch.int32, device=dev)
        self.top_w = torch.empty(T, K, dtype=torch.float32, device=dev)
        self.compute = _CODE[w.act] if w.act in ("bf16", "f16") else _lib.QW_BF16
        self.ws_bytes = _lib.load().qw_moe_decode_step_workspace_bytes(T, w.d_model, E, K, w.d_ff, self.compute)
        self.ws = _hip.workspace(self.ws_bytes, dev)
        self._fn = _lib.load().qw_moe_decode_step
        self._head = [_hip.ptr(self.x), _hip.ptr(self.residual), T, w.d_model, _hip.ptr(self.router), 1.0,
                      _hip.ptr(layer.bias), E, K, w.d_ff, self.compute, *layer.weight_args(), _hip.ptr(self.out),
                      _hip.ptr(self.probs), _hip.ptr(self.top_idx), _hip.ptr(self.top_w), _hip.ptr(self.ws),
                      self.ws_bytes]

    def __call__(self) -> None:
        st = self._fn(*self._head, _hip.stream(self.x.device))
        if st:
            _lib.check(st, "qw_moe_decode_step")


def module_from_layer(layer: Layer):
    """A TopKMoE module holding this layer's router and experts (the drop-in
    surface the reference's callers use), on the layer's device."""
    from .moe import QuantaWeaveConfig, TopKMoE
    from .quantization import QuantizedLinear

    w = layer.w
    cfg = QuantaWeaveConfig(vocab_size=2, hidden_size=w.d_model, layers=1, ffn_size=w.d_ff, num_experts=w.experts,
                            top_k=w.top_k, attention_heads=1, capacity_factor=w.capacity_factor)
    dev = layer.x.device
    moe = TopKMoE(cfg).to(device=dev, dtype=layer.x.dtype)
    with torch.no_grad():
        moe.router.weight.copy_(layer.router)
        for e, expert in enumerate(moe.experts):
            for name in ("gate", "up", "down"):
                stored = getattr(layer, name)[e]
                if layer.fmt in (_lib.QW_F32, _lib.QW_BF16, _lib.QW_F16):
                    getattr(expert, name).weight.copy_(stored)
                    continue
                lin = getattr(expert, name)
                bits = 8 if layer.fmt == _lib.QW_I8 else 4
                group = layer.group_ff if name == "down" else layer.group_in
                q = QuantizedLinear(lin.in_features, lin.out_features, bits, group).to(dev)
                q.qweight.copy_(stored)
                q.scales.copy_(getattr(layer, name + "_s")[e])
                setattr(expert, name, q)
    moe.expert_bias = layer.bias
    moe.requires_grad_(False)
    return moe
