"""Gradient oracle for the grouped expert matmuls and the MoE layer — TEST
INFRASTRUCTURE ONLY (imported by ``tests/`` alone).

The reference differentiates its forward with torch autograd.  This module
restates that forward in float64 on the CPU with plain torch ops and lets
autograd differentiate it; the gradients are then those of the mathematics,
up to float64 rounding.  Routing decisions (top-k indices, the capacity
plan) are inputs, taken from the run under test: they are pinned bit for bit
by the forward oracle and are piecewise constant, so they carry no gradient.
"""

from __future__ import annotations

from typing import Sequence

import torch
import torch.nn.functional as F
from torch import Tensor


def grouped_matmul(x: Tensor, weight: Tensor, counts: Sequence[int]) -> Tensor:
    """Per-expert x @ W[e]^T over consecutive row blocks — the loop the
    reference's kernel test compares against (tests/test_moe_kernels.py:16-21)
    for grouped_matmul (src/moe_kernels.py:167-171)."""
    outs, start = [], 0
    for e, c in enumerate(counts):
        outs.append(x[start:start + c] @ weight[e].t())
        start += c
    return torch.cat(outs) if outs else x.new_zeros(0, weight.size(1))


def swiglu(x: Tensor, gate: Tensor, up: Tensor, down: Tensor) -> Tensor:
    """SparseSwiGLU.forward (src/quantweave_moe_model.py:59-60) with weights in
    nn.Linear [out, in] layout."""
    return F.linear(F.silu(F.linear(x, gate)) * F.linear(x, up), down)


def grouped_swiglu(x: Tensor, gate: Tensor, up: Tensor, down: Tensor, counts: Sequence[int]) -> Tensor:
    """The per-expert loop grouped_swiglu replaces (src/moe_kernels.py:186-195,
    tests/test_moe_kernels.py:71-76); gate/up/down stacked [E, out, in]."""
    outs, start = [], 0
    for e, c in enumerate(counts):
        outs.append(swiglu(x[start:start + c], gate[e], up[e], down[e]))
        start += c
    return torch.cat(outs) if outs else x.new_zeros(0, down.size(1))


def moe_layer(x: Tensor, router_w: Tensor, gate: Tensor, up: Tensor, down: Tensor, top_idx: Tensor,
              kept: Tensor, temperature: float = 1.0) -> tuple[Tensor, Tensor, Tensor]:
    """TopKMoE.forward (src/quantweave_moe_model.py:123-154) given its routing.

    x [T, D]; router_w [E, D]; gate/up [E, F, D], down [E, D, F];
    top_idx [T, K] the selected experts (expert_bias only steers this choice);
    kept [T, K] bool, the routes the capacity plan keeps (:166-188).
    Returns (output [T, D], router_probs [T, E], balance_loss).  Every
    operation is differentiable in float64: the softmax (:126-127), the
    gather and renormalisation of the top-k weights (:133-135), the experts
    on their kept rows weighted and index-added (:190-202), and the balance
    loss (:152-154)."""
    T, K = top_idx.shape
    E = router_w.size(0)
    logits = F.linear(x, router_w) / temperature
    probs = logits.softmax(dim=-1)
    w = probs.gather(1, top_idx)
    w = w / w.sum(dim=-1, keepdim=True)
    out = torch.zeros_like(x)
    for e in range(E):
        sel = (top_idx == e) & kept
        tokens = sel.nonzero()[:, 0]
        if tokens.numel() == 0:
            continue
        rows = swiglu(x[tokens], gate[e], up[e], down[e]) * w[sel][:, None]
        out = out.index_add(0, tokens, rows)
    importance = probs.mean(dim=0)
    assignments = F.one_hot(top_idx, E).to(x.dtype).mean(dim=(0, 1))
    balance = E * (importance * assignments).sum()
    return out, probs, balance


def kept_routes(top_idx: Tensor, dropped_token: Tensor, dropped_expert: Tensor, n_dropped: int) -> Tensor:
    """[T, K] bool: True where route (t, j) was not dropped by the plan."""
    kept = torch.ones(top_idx.shape, dtype=torch.bool)
    for t, e in zip(dropped_token[:n_dropped].tolist(), dropped_expert[:n_dropped].tolist()):
        kept[t] &= top_idx[t] != e
    return kept
