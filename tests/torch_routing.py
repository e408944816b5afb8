"""The reference's routing composition run by torch itself (tests only).

The reference routes with torch's library calls (src/quantweave_moe_model.py:
127-136 for the layer, :172-188 for the plan; src/fast_decode.py:170-174 for
the decode step).  Run on the GPU these are the bits the reference produces on
this device, which the library must reproduce; run on the CPU they pin the
oracle's selection and plan.
"""

import numpy as np
import torch


def torch_route(logits: torch.Tensor, k: int, bias: torch.Tensor | None = None, select: str = "probs"):
    """softmax -> topk (or biased topk + gather) -> renormalise, on the
    tensors' device.  select="logits" is the decode step's top-k of the
    scores.  Returns (probs, top_idx int64, top_w)."""
    probs = logits.softmax(dim=-1)
    if bias is None and select == "probs":
        top_w, top_idx = probs.topk(k, dim=-1)
    else:
        scores = logits if bias is None else logits + bias.to(logits)
        top_idx = scores.topk(k, dim=-1).indices
        top_w = probs.gather(1, top_idx)
    top_w = top_w / top_w.sum(dim=-1, keepdim=True)
    return probs, top_idx, top_w


def torch_plan(top_idx: torch.Tensor, top_w: torch.Tensor, experts: int, capacity: int):
    """TopKMoE._plan's double stable argsort, on the tensors' device."""
    k = top_idx.shape[1]
    route_experts = top_idx.long().reshape(-1)
    route_weights = top_w.reshape(-1)
    by_weight = torch.argsort(route_weights, descending=True, stable=True)
    order = by_weight[torch.argsort(route_experts[by_weight], stable=True)]
    counts = torch.bincount(route_experts, minlength=experts)
    offsets = torch.cumsum(counts, dim=0) - counts
    position = torch.arange(order.numel(), device=order.device) - offsets[route_experts[order]]
    keep = position < capacity
    kept, dropped = order[keep], order[~keep]
    return dict(tokens=kept // k, weights=route_weights[kept], kept_counts=counts.clamp(max=capacity),
                overflow=int((~keep).sum()), dropped_tokens=dropped // k, dropped_experts=route_experts[dropped],
                counts=counts)


def assert_plan_equal(got: dict, ref: dict):
    """A plan from the C ABI (numpy arrays, tests/hipcall.plan) against torch_plan."""
    cpu = {k: (v.cpu().numpy() if isinstance(v, torch.Tensor) else v) for k, v in ref.items()}
    assert np.array_equal(got["slot_token"], cpu["tokens"]), "capacity slots differ"
    assert np.array_equal(got["slot_weight"].view(np.int32), cpu["weights"].view(np.int32)), "slot weights differ"
    assert np.array_equal(got["kept_counts"], cpu["kept_counts"])
    assert np.array_equal(got["counts"], cpu["counts"])
    assert int(got["totals"][1]) == cpu["overflow"], "overflow differs"
    assert np.array_equal(got["dropped_token"], cpu["dropped_tokens"]), "dropped tokens differ"
    assert np.array_equal(got["dropped_expert"], cpu["dropped_experts"]), "dropped experts differ"
