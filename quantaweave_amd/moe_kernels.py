"""Grouped expert kernels — drop-in for QuantaWeave's moe_kernels.py on MI355X.

Same public names and argument meaning as src/moe_kernels.py:
``kernels_available``, ``experts_support_grouped``, ``GroupedPlan``,
``grouped_matmul``, ``compute_dtype``, ``grouped_swiglu`` and ``benchmark``.
The kernels are hand-written HIP for gfx950 behind the C ABI
(include/qwmoe.h), forward and backward.  Differences from the reference:

* quantised experts (``QuantizedLinear``) are supported by the grouped path
  (the reference restricts it to nn.Linear, src/moe_kernels.py:174-176);
* the tile schedule is built on the device from per-expert row offsets, so
  ``GroupedPlan`` only carries those offsets (plus the reference's ``tiles`` /
  ``rows`` bookkeeping);
* expert weights are stacked once and cached, not re-stacked per call.
"""

from __future__ import annotations

import time
from typing import Optional, Sequence

import torch
from torch import Tensor, nn

from . import _hip, _lib
from .moe import packed_experts
from .quantization import QuantizedLinear

BLOCK_M = 32  # row-tile height used for the reference's `tiles` count


def kernels_available(device: torch.device) -> bool:
    """True when the HIP library is built and `device` is a ROCm device (src/moe_kernels.py:34-35)."""
    device = torch.device(device)
    return _lib.available() and device.type == "cuda" and torch.cuda.is_available() and torch.version.hip is not None


class GroupedPlan:
    """Row blocks of expert-sorted rows (src/moe_kernels.py:92-111)."""

    def __init__(self, counts: Sequence[int], device: torch.device) -> None:
        counts = [int(c) for c in counts]
        if any(c < 0 for c in counts):
            raise ValueError("counts must be non-negative")
        offsets, total = [0], 0
        for c in counts:
            total += c
            offsets.append(total)
        self.tiles = sum(-(-c // BLOCK_M) for c in counts)
        self.rows = total
        self.num_experts = len(counts)
        self.counts = counts
        self.max_count = max(counts, default=0)
        self.offsets = torch.tensor(offsets, dtype=torch.int32, device=device)


def experts_support_grouped(experts: nn.ModuleList) -> bool:
    """Bias-free nn.Linear experts (src/moe_kernels.py:174-176) or QuantizedLinear experts of one format."""
    def ok(p) -> bool:
        return isinstance(p, QuantizedLinear) or (isinstance(p, nn.Linear) and p.bias is None)

    return all(ok(getattr(e, name, None)) for e in experts for name in ("gate", "up", "down"))


def compute_dtype(inputs: Tensor) -> torch.dtype:
    """The autocast dtype when autocast is on, else the input dtype (src/moe_kernels.py:179-183)."""
    device_type = inputs.device.type
    if torch.is_autocast_enabled(device_type):
        return torch.get_autocast_dtype(device_type)
    return inputs.dtype


def _check_operands(x: Tensor, weight: Tensor, plan: GroupedPlan, what: str) -> int:
    _hip.require_device(x, what)
    act = _hip.act_code(x, what)
    if weight.dim() != 3 or weight.size(0) != plan.num_experts or weight.size(2) != x.size(1):
        raise ValueError("weight must be [experts, out, in] matching the plan and x")
    if x.size(0) != plan.rows:
        raise ValueError(f"x has {x.size(0)} rows but the plan covers {plan.rows}")
    return act


def _forward(x: Tensor, w: Tensor, plan: GroupedPlan, act: int) -> Tensor:
    """out[rows of e] = x[rows of e] @ w[e]^T; x, w contiguous of one dtype."""
    out = torch.empty(x.size(0), w.size(1), dtype=x.dtype, device=x.device)
    if x.size(0):
        _lib.call("qw_grouped_matmul", _hip.ptr(x), act, _hip.ptr(w), act, None, 0, w.size(0), w.size(1), w.size(2),
                  _hip.ptr(plan.offsets), x.size(0), plan.max_count, _hip.ptr(out), _hip.stream(x.device))
    return out


def _backward(grad: Tensor, x: Tensor, w: Tensor, plan: GroupedPlan, act: int, need_x: bool, need_w: bool,
              grad_x: Optional[Tensor] = None, grad_w_dtype: Optional[torch.dtype] = None
              ) -> tuple[Optional[Tensor], Optional[Tensor]]:
    """(grad_x, grad_w) of out = grouped x @ w^T.  A given grad_x is added to.
    grad_w_dtype: float32 to get the weight gradient unrounded (fp32
    parameters multiplied in bf16); default the operands' dtype."""
    gx = gw = None
    accumulate = grad_x is not None
    if need_x:
        gx = grad_x if accumulate else torch.empty_like(x)
    gw_dtype = w.dtype if grad_w_dtype is None else grad_w_dtype
    if need_w:
        gw = torch.empty(w.shape, dtype=gw_dtype, device=w.device)
    if gx is not None or gw is not None:
        nbytes = _lib.load().qw_grouped_matmul_backward_workspace_bytes(w.size(0), w.size(1), w.size(2), x.size(0), act)
        ws = _hip.workspace(nbytes, x.device)
        _lib.call("qw_grouped_matmul_backward", _hip.ptr(grad), _hip.ptr(x), _hip.ptr(w), act, w.size(0), w.size(1),
                  w.size(2), _hip.ptr(plan.offsets), x.size(0), plan.max_count, _hip.ptr(gx), int(accumulate),
                  _hip.ptr(gw), _hip.act_code(torch.empty(0, dtype=gw_dtype), "grad_w"), _hip.ptr(ws), nbytes,
                  _hip.stream(x.device))
    return gx, gw


class _GroupedMatmul(torch.autograd.Function):
    """src/moe_kernels.py:138-164: grad_x = grad_out @ W[e] per expert block,
    grad_W[e] = grad_out[rows of e]^T @ x[rows of e] (exactly zero for an
    expert without rows), both through qw_grouped_matmul_backward."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, plan: GroupedPlan) -> Tensor:
        act = _check_operands(x, weight, plan, "grouped_matmul")
        x = x.contiguous()
        w = weight.detach().to(x.dtype).contiguous()
        ctx.save_for_backward(x, w)
        ctx.plan, ctx.act, ctx.weight_dtype = plan, act, weight.dtype
        return _forward(x, w, plan, act)

    @staticmethod
    def backward(ctx, grad_output: Tensor):
        x, w = ctx.saved_tensors
        grad = grad_output.contiguous().to(x.dtype)
        gx, gw = _backward(grad, x, w, ctx.plan, ctx.act, ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        if gw is not None:
            gw = gw.to(ctx.weight_dtype)
        return gx, gw, None


def grouped_matmul(x: Tensor, weight: Tensor, plan: GroupedPlan) -> Tensor:
    """Per-expert x @ W[e]^T over expert-sorted rows; weight is [E, out, in] (src/moe_kernels.py:167-171).

    Differentiable in x and weight (the backward runs the grouped HIP kernels)."""
    return _GroupedMatmul.apply(x, weight, plan)


class _GroupedSwiGLU(torch.autograd.Function):
    """down(silu(gate(x)) * up(x)) over expert blocks with its backward, the
    composition grouped_swiglu builds from _GroupedMatmul and F.silu
    (src/moe_kernels.py:186-195): three grouped matmuls and qw_swiglu forward;
    qw_swiglu_backward and five grouped backward products (grad_x of gate and
    up summed in place) backward.  Weights are stacked [E, out, in] of x's dtype."""

    @staticmethod
    def forward(ctx, x: Tensor, gate: Tensor, up: Tensor, down: Tensor, plan: GroupedPlan) -> Tensor:
        act = _hip.act_code(x, "grouped_swiglu")
        x = x.contiguous()
        gate, up, down = (t.detach().contiguous() for t in (gate, up, down))
        g = _forward(x, gate, plan, act)
        u = _forward(x, up, plan, act)
        h = torch.empty_like(g)
        _lib.call("qw_swiglu", _hip.ptr(g), _hip.ptr(u), act, g.numel(), _hip.ptr(h), _hip.stream(x.device))
        y = _forward(h, down, plan, act)
        ctx.save_for_backward(x, gate, up, down, g, u, h)
        ctx.plan, ctx.act = plan, act
        return y

    @staticmethod
    def backward(ctx, grad_output: Tensor):
        x, gate, up, down, g, u, h = ctx.saved_tensors
        plan, act = ctx.plan, ctx.act
        need_x, need_g, need_u, need_d = ctx.needs_input_grad[:4]
        grad = grad_output.contiguous().to(x.dtype)
        dh, d_down = _backward(grad, h, down, plan, act, True, need_d)
        dg, du = torch.empty_like(g), torch.empty_like(u)
        _lib.call("qw_swiglu_backward", _hip.ptr(dh), _hip.ptr(g), _hip.ptr(u), act, g.numel(), _hip.ptr(dg),
                  _hip.ptr(du), _hip.stream(x.device))
        dx, d_gate = _backward(dg, x, gate, plan, act, need_x, need_g)
        dx, d_up = _backward(du, x, up, plan, act, need_x, need_u, grad_x=dx)
        return dx, d_gate, d_up, d_down, None


def _needs_grad(inputs: Tensor, experts: nn.ModuleList) -> bool:
    if not torch.is_grad_enabled():
        return False
    return inputs.requires_grad or any(p.requires_grad for p in experts.parameters())


def grouped_swiglu(inputs: Tensor, experts: nn.ModuleList, counts: Sequence[int], plan: Optional[GroupedPlan] = None) -> Tensor:
    """SwiGLU over expert-sorted rows: down(silu(gate(x)) * up(x)) with each
    expert's own weights (src/moe_kernels.py:186-195).

    Without gradients: one pair of HIP kernels (fused gate/up + SiLU·mul, then
    down) on the cached expert stacks.  With gradients (autograd on and the
    inputs or expert weights requiring grad): the differentiable composition
    over freshly stacked weights, as the reference stacks them per call."""
    _hip.require_device(inputs, "grouped_swiglu")
    plan = plan or GroupedPlan(counts, inputs.device)
    if plan.num_experts != len(experts):
        raise ValueError("plan and experts disagree on the number of experts")
    dtype = compute_dtype(inputs)
    if inputs.size(0) != plan.rows:
        raise ValueError(f"inputs have {inputs.size(0)} rows but the plan covers {plan.rows}")
    if _needs_grad(inputs, experts):
        if any(isinstance(getattr(e, n), QuantizedLinear) for e in experts for n in ("gate", "up", "down")):
            raise NotImplementedError("gradients through quantised experts are not supported")
        x = inputs.to(dtype)
        _hip.act_code(x, "grouped_swiglu")
        gate = torch.stack([e.gate.weight for e in experts]).to(dtype)
        up = torch.stack([e.up.weight for e in experts]).to(dtype)
        down = torch.stack([e.down.weight for e in experts]).to(dtype)
        return _GroupedSwiGLU.apply(x, gate, up, down, plan)
    x = inputs.detach().to(dtype).contiguous()
    act = _hip.act_code(x, "grouped_swiglu")
    pack = packed_experts(experts, experts)
    # the reference casts the stacked weights to the compute dtype (src/moe_kernels.py:191-193);
    # bf16 weights under fp32 activations are widened exactly inside the kernels
    args = pack.args_for(act)
    d_ff = pack.gate.size(1)
    d_model = x.size(1)
    out = torch.empty(plan.rows, d_model, dtype=dtype, device=x.device)
    if plan.rows:
        lib = _lib.load()
        nbytes = lib.qw_moe_experts_workspace_bytes(plan.rows, len(experts), d_model, d_ff, act)
        ws = _hip.workspace(nbytes, x.device)
        _lib.call("qw_moe_experts", _hip.ptr(x), act, None, _hip.ptr(plan.offsets), len(experts), d_model, d_ff,
                  plan.rows, max(plan.counts), *args, None, _hip.ptr(out), _hip.ptr(ws), nbytes, _hip.stream(x.device))
    return out


def benchmark(experts: int = 32, tokens: int = 8192, hidden: int = 256, ffn: int = 512, top_k: int = 2, repeats: int = 20,
              bf16: bool = False) -> dict:
    """Wall-clock the loop and grouped expert paths on the current GPU
    (forward + backward), optionally under bf16 autocast (src/moe_kernels.py:
    198-227): ``loop_ms`` is the per-expert executor (``use_triton_kernels =
    False``), ``triton_ms`` the grouped one, ``speedup`` their ratio; both run
    the HIP kernels.  ``forward_ms`` (not in the reference) is the grouped
    forward alone under no_grad."""
    from .moe import QuantaWeaveConfig, TopKMoE

    if not kernels_available(torch.device("cuda")):
        raise RuntimeError("benchmark needs a ROCm device and the built HIP library")
    config = QuantaWeaveConfig(vocab_size=8, hidden_size=hidden, layers=1, ffn_size=ffn, num_experts=experts, top_k=top_k,
                               attention_heads=1, max_sequence_length=tokens, capacity_factor=0)
    moe = TopKMoE(config).cuda()
    x = torch.randn(1, tokens, hidden, device="cuda", requires_grad=True)

    def context():
        return torch.autocast("cuda", dtype=torch.bfloat16) if bf16 else torch.autocast("cuda", enabled=False)

    def train_step():
        with context():
            out = moe(x)[0]
        out.float().sum().backward()

    def forward():
        with torch.no_grad(), context():
            moe(x)

    result = {}
    for name, fn, grouped in (("loop", train_step, False), ("triton", train_step, True), ("forward", forward, True)):
        moe.use_triton_kernels = grouped
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        started = time.perf_counter()
        for _ in range(repeats):
            fn()
        torch.cuda.synchronize()
        result[name + "_ms"] = (time.perf_counter() - started) / repeats * 1000
    result["speedup"] = result["loop_ms"] / result["triton_ms"]
    result.update(experts=experts, tokens=tokens, hidden=hidden, ffn=ffn, top_k=top_k, bf16=bf16)
    return result


if __name__ == "__main__":
    # src/moe_kernels.py:230-235: print the benchmark as JSON
    import argparse
    import json

    ap = argparse.ArgumentParser(description="forward + backward wall clock of the loop and grouped executors")
    ap.add_argument("--experts", type=int, default=32)
    ap.add_argument("--tokens", type=int, default=8192)
    ap.add_argument("--hidden", type=int, default=256)
    ap.add_argument("--ffn", type=int, default=512)
    ap.add_argument("--top-k", type=int, default=2)
    ap.add_argument("--repeats", type=int, default=20)
    ap.add_argument("--bf16", action="store_true", help="under bf16 autocast")
    a = ap.parse_args()
    print(json.dumps(benchmark(a.experts, a.tokens, a.hidden, a.ffn, a.top_k, a.repeats, a.bf16)), flush=True)
