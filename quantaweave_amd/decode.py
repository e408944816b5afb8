"""One-token MoE step for incremental decoding — the routed-expert part of
QuantaWeave's ``FastDecoder`` (src/fast_decode.py).

``FastDecoder`` reads each layer's router and experts once at construction
(src/fast_decode.py:117-123, dequantising int8/int4 experts into dense stacks
via ``layer_weight``, :64-73) and evaluates the MoE block of every step with
fp32 routing, no capacity and one einsum per projection (:170-177).
``MoEDecodeStep`` does the same step as one call into the C ABI
(``qw_moe_decode_step``): the experts stay in their stored format (int4/int8
packed, or bf16/fp32), and only the routed experts' weights are read.  All
buffers are allocated at construction, so a call can be recorded in a
``torch.cuda.CUDAGraph`` and replayed, as FastDecoder records its step
(:178-204).
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor, nn

from . import _hip, _lib
from .moe import ExpertPack


def precision_dtype(device: torch.device, precision: str) -> torch.dtype:
    """src/fast_decode.py:75-78: "auto" is bf16 on a GPU; "bf16", "fp16" and
    "fp32" name their dtypes."""
    if precision == "auto":
        precision = "bf16" if device.type == "cuda" else "fp32"
    return {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[precision]


class MoEDecodeStep:
    """The routed experts of one layer for ``tokens`` rows at a time.

    ``moe`` is a ``TopKMoE`` (this package's or the reference's: anything with
    ``router``, ``experts[i].{gate,up,down}``, ``top_k``,
    ``router_temperature`` and ``expert_bias``).  Float experts are cast to
    the compute dtype once, as ``layer.gate = stack(...).to(dtype)`` does
    (src/fast_decode.py:121-123); quantised experts keep their packed bytes.

    ``step(normed, residual)`` returns ``residual + sum_j y_j * w_j`` in fp32
    (src/fast_decode.py:177), written to ``out`` (default: a buffer owned by
    this object, reused by every call).  ``last_top_indices`` and
    ``last_top_weights`` hold the routing of the last call.
    """

    def __init__(self, moe: nn.Module, device: Optional[torch.device] = None, precision: str = "auto",
                 tokens: int = 1) -> None:
        router = moe.router.weight.detach()
        device = torch.device(device) if device is not None else router.device
        _hip.require_device(torch.empty(0, device=device), "MoEDecodeStep")
        self.device = device
        self.dtype = precision_dtype(device, precision)
        self.compute = _hip.act_code(torch.empty(0, dtype=self.dtype), "MoEDecodeStep")
        self.tokens = int(tokens)
        if self.tokens < 1:
            raise ValueError("tokens must be positive")
        self.router = router.to(device, torch.float32).contiguous()               # routing stays fp32
        self.experts_count, self.hidden = self.router.shape
        self.top_k = int(moe.top_k)
        if not 1 <= self.top_k <= self.experts_count:
            raise ValueError("top_k must be between 1 and num_experts")
        self.temperature = float(moe.router_temperature)
        if self.temperature <= 0:
            raise ValueError("router_temperature must be positive")
        bias = getattr(moe, "expert_bias", None)
        self.bias = None if bias is None else bias.detach().to(device, torch.float32).contiguous()
        experts = moe.experts
        pack = ExpertPack(experts, rehome=False)
        for name in ("gate", "up", "down", "gate_s", "up_s", "down_s"):
            t = getattr(pack, name)
            if t is not None:
                setattr(pack, name, t.to(device).contiguous())
        pack.maybe_tile()
        # float experts in another 16-bit compute type: one cast copy (tiled where the shapes allow)
        self.pack = pack.for_act(self.compute)
        self.ffn = int(experts[0].gate.out_features)
        T, E, K = self.tokens, self.experts_count, self.top_k
        lib = _lib.load()
        self.ws_bytes = lib.qw_moe_decode_step_workspace_bytes(T, self.hidden, E, K, self.ffn, self.compute)
        self.workspace = _hip.workspace(self.ws_bytes, device)
        self.out = torch.empty(T, self.hidden, dtype=torch.float32, device=device)
        self.probs = torch.empty(T, E, dtype=torch.float32, device=device)
        self.last_top_indices = torch.empty(T, K, dtype=torch.int32, device=device)
        self.last_top_weights = torch.empty(T, K, dtype=torch.float32, device=device)

    def _check(self, t: Tensor, what: str) -> None:
        if t.device != self.device or t.dtype != torch.float32 or tuple(t.shape) != (self.tokens, self.hidden) \
                or not t.is_contiguous():
            raise ValueError(f"{what} must be a contiguous fp32 [{self.tokens}, {self.hidden}] tensor on {self.device}")

    def step(self, normed: Tensor, residual: Optional[Tensor] = None, out: Optional[Tensor] = None) -> Tensor:
        self._check(normed, "normed")
        if residual is not None:
            self._check(residual, "residual")
        out = self.out if out is None else out
        self._check(out, "out")
        _lib.call("qw_moe_decode_step", _hip.ptr(normed), _hip.ptr(residual), self.tokens, self.hidden,
                  _hip.ptr(self.router), self.temperature, _hip.ptr(self.bias), self.experts_count, self.top_k,
                  self.ffn, self.compute, *self.pack.args(), _hip.ptr(out), _hip.ptr(self.probs),
                  _hip.ptr(self.last_top_indices), _hip.ptr(self.last_top_weights), _hip.ptr(self.workspace),
                  self.ws_bytes, _hip.stream(self.device))
        return out

    __call__ = step

    def scores(self) -> Tensor:
        """The router scores (fp32 [tokens, experts], after the temperature) of
        the last call: the first region of the workspace, as qw_moe_decode_step
        lays it out."""
        n = self.tokens * self.experts_count * 4
        return self.workspace[:n].view(torch.float32).view(self.tokens, self.experts_count)
