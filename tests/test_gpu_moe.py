"""Whole MoE layer forward on the GPU (qw_moe_forward / TopKMoE) against the oracle.

Routing (probabilities against torch's softmax on the device; indices,
weights, capacity slots, drops, overflow against the oracle fed those
probabilities) is compared bit for bit given the kernel's logits; outputs normwise within 1e-4 (fp32) or
2e-2 (bf16 / int8 / int4).  Each workload runs at an oracle-friendly scale and
at its full size.
"""

import numpy as np
import pytest
import torch

import oracle
import quantaweave_amd as qa
from quantaweave_amd import workloads as W

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-4, "bf16": 2e-2, "f16": 5e-3}


def normwise(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)


# Elementwise relative error at the 99.9th percentile, with an absolute floor
# of the normwise tolerance times the output's largest magnitude (below it, a
# sum whose terms cancel has no relative accuracy to speak of in bf16): a
# second view of the same outputs next to the normwise bound.
P999 = {"f32": 1e-3, "bf16": 0.5, "f16": 0.1}


def elementwise_p999(got, ref, dtype):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    floor = TOL[dtype] * max(np.abs(ref).max(), 1e-30)
    return float(np.percentile(np.abs(got - ref) / np.maximum(np.abs(ref), floor), 99.9))


def host_weights(layer):
    w = layer.w
    fmt = w.weights
    out = dict(format=fmt, d_model=w.d_model, d_ff=w.d_ff, group_in=layer.group_in, group_ff=layer.group_ff)
    for name in ("gate", "up", "down"):
        t = getattr(layer, name)
        out[name] = t.float().cpu().numpy() if fmt in ("f32", "bf16", "f16") else t.cpu().numpy()
        s = getattr(layer, name + "_s")
        if s is not None:
            out[name + "_scales"] = s.cpu().numpy()
    return out


def check_layer(workload, tol_scale=1.0, tiles=False):
    print(f"case {workload.name} T={workload.tokens} d={workload.d_model} E={workload.experts} f={workload.d_ff}"
          f"{' tiled' if tiles else ''}", flush=True)
    layer = W.build_layer(workload)
    if tiles:
        layer.add_tiles()
        assert "tiles" in layer.extra
    run = W.LayerRunner(layer)
    run()
    torch.cuda.synchronize()
    logits = run.workspace_view("logits").cpu().numpy()
    x = layer.x.float().cpu().numpy()
    rw = layer.router.float().cpu().numpy()
    # router logits within fp32 accumulation error of the double-precision oracle
    ref_logits = oracle.router_logits(x, rw)
    assert np.abs(logits - ref_logits).max() <= 1e-5 * max(1.0, np.abs(ref_logits).max())
    bias = None if layer.bias is None else layer.bias.cpu().numpy()
    # the probabilities are torch's softmax on this device, bit for bit
    probs_t = torch.softmax(run.workspace_view("logits"), dim=-1)
    assert torch.equal(run.probs, probs_t)
    res = oracle.moe_forward(x, rw, host_weights(layer), top_k=workload.top_k, cap=run.capacity, dtype=workload.act,
                             expert_bias=bias, logits=logits, probs=probs_t.cpu().numpy())
    # bit-exact routing and plan
    assert np.array_equal(run.probs.cpu().numpy().view(np.int32), res["probs"].view(np.int32))
    assert np.array_equal(run.top_idx.cpu().numpy(), res["top_idx"])
    assert np.array_equal(run.top_w.cpu().numpy().view(np.int32), res["top_w"].view(np.int32))
    p = res["plan"]
    assert np.array_equal(run.counts.cpu().numpy(), p["counts"])
    assert np.array_equal(run.kept_counts.cpu().numpy(), p["kept_counts"])
    assert run.totals.cpu().tolist() == p["totals"].tolist()
    kept, nd = int(p["totals"][0]), int(p["totals"][1])
    assert np.array_equal(run.workspace_view("slot_token").cpu().numpy()[:kept], p["slot_token"])
    assert np.array_equal(run.workspace_view("route_slot").cpu().numpy(), p["route_slot"])
    assert np.array_equal(run.dropped_token.cpu().numpy()[:nd], p["dropped_token"])
    assert np.array_equal(run.dropped_expert.cpu().numpy()[:nd], p["dropped_expert"])
    # expert outputs
    got = run.out.float().cpu().numpy()
    assert np.isfinite(got).all()
    nw = normwise(got, res["out"])
    p999 = elementwise_p999(got, res["out"], workload.act)
    print(f"  normwise {nw:.3e}  elementwise p99.9 {p999:.3e}", flush=True)
    assert nw <= TOL[workload.act] * tol_scale
    assert p999 <= P999[workload.act] * tol_scale
    return run, res


SMALL = [
    W.WORKLOADS["fp32-plumbing-T512-d256-E8-f512-k2"],
    W.scaled(W.WORKLOADS["bf16-prefill-T8192-d2048-E64-f1024-k2"], tokens=1024, d_model=512, d_ff=256),
    W.scaled(W.WORKLOADS["int8-decode-T64-d2048-E64-f1024-k2"], d_model=512, d_ff=256),
    W.scaled(W.WORKLOADS["int4-decode-T16-d4096-E64-f1408-k2"], d_model=1024, d_ff=352),
    W.scaled(W.WORKLOADS["skewed-T4096-d2048-E64-f1024-k2"], tokens=1024, d_model=512, d_ff=256),
    W.scaled(W.WORKLOADS["int8-prefill-T8192-d2048-E64-f1024-k2"], tokens=2048, d_model=512, d_ff=256, experts=8),
    W.scaled(W.WORKLOADS["int4-prefill-T8192-d2048-E64-f1024-k2"], tokens=2048, d_model=512, d_ff=256, experts=8),
]


@pytest.mark.parametrize("workload", SMALL, ids=lambda w: w.name)
def test_layer_matches_oracle_small(workload):
    run, res = check_layer(workload)
    if workload.capacity_factor == 1.0:
        assert int(res["plan"]["totals"][1]) > 0            # the skewed workload drops routes


@pytest.mark.parametrize("name", [n for n in W.WORKLOADS if not n.startswith("fp32")])
def test_layer_matches_oracle_full_size(name):
    check_layer(W.WORKLOADS[name])


@pytest.mark.parametrize("name", ["bf16-prefill-T8192-d2048-E64-f1024-k2", "skewed-T4096-d2048-E64-f1024-k2"])
def test_layer_matches_oracle_full_size_tiled(name):
    """The weights in the QW_BF16T tiles the module (and the benchmark) uses:
    the exact kernel instantiations behind the benchmark figures."""
    check_layer(W.WORKLOADS[name], tiles=True)


def f16_workload(name: str, **sizes) -> W.Workload:
    """A workload with fp16 activations (and fp16 weights where it has 16-bit ones)."""
    base = W.WORKLOADS[name]
    small = W.scaled(base, **sizes) if sizes else base
    return W.Workload(small.name.replace("bf16", "f16") + "-f16", small.tokens, small.d_model, small.experts,
                      small.d_ff, small.top_k, small.capacity_factor, "f16",
                      "f16" if small.weights == "bf16" else small.weights, small.seed, small.group_size, small.zipf)


F16_CASES = [
    (f16_workload("bf16-prefill-T8192-d2048-E64-f1024-k2", tokens=1024, d_model=512, d_ff=256), False),
    (f16_workload("bf16-prefill-T8192-d2048-E64-f1024-k2"), True),
    (f16_workload("int8-decode-T64-d2048-E64-f1024-k2"), False),
    (f16_workload("int4-decode-T16-d4096-E64-f1408-k2"), False),
    (f16_workload("int4-prefill-T8192-d2048-E64-f1024-k2", tokens=2048, d_model=512, d_ff=256, experts=8), False),
    (f16_workload("skewed-T4096-d2048-E64-f1024-k2", tokens=1024, d_model=512, d_ff=256), True),
]


@pytest.mark.parametrize("workload,tiles", F16_CASES, ids=lambda v: v.name if hasattr(v, "name") else str(v))
def test_layer_matches_oracle_f16(workload, tiles):
    """fp16 activations and weights (the reference's fp16 precision): the
    matrix-core, weight-streaming and quantised paths in fp16 against the
    oracle with fp16 rounding points."""
    check_layer(workload, tiles=tiles)


def test_layer_is_deterministic_across_calls():
    layer = W.build_layer(W.scaled(W.WORKLOADS["skewed-T4096-d2048-E64-f1024-k2"], tokens=2048, d_model=512, d_ff=256))
    run = W.LayerRunner(layer)
    run()
    first = (run.out.clone(), run.top_idx.clone(), run.workspace_view("slot_token").clone())
    for _ in range(3):
        run()
    torch.cuda.synchronize()
    assert torch.equal(first[0], run.out) and torch.equal(first[1], run.top_idx)
    assert torch.equal(first[2], run.workspace_view("slot_token"))


# ---------------------------------------------------------------- the TopKMoE module surface
def small_config(**overrides):
    values = dict(vocab_size=32, hidden_size=16, layers=2, ffn_size=32, num_experts=6, top_k=2,
                  attention_heads=2, max_sequence_length=16, capacity_factor=0, min_expert_capacity=1)
    values.update(overrides)
    return qa.QuantaWeaveConfig(**values)


def module_weights(moe):
    return dict(format="f32", d_model=moe.router.in_features, d_ff=moe.experts[0].gate.out_features,
                gate=np.stack([e.gate.weight.detach().cpu().numpy() for e in moe.experts]),
                up=np.stack([e.up.weight.detach().cpu().numpy() for e in moe.experts]),
                down=np.stack([e.down.weight.detach().cpu().numpy() for e in moe.experts]))


@pytest.mark.parametrize("capacity_factor", [0, 0.6])
def test_topkmoe_matches_oracle_and_reports_overflow(capacity_factor):
    # tests/test_model_features.py:38-46
    torch.manual_seed(0)
    moe = qa.TopKMoE(small_config(capacity_factor=capacity_factor, min_expert_capacity=2)).cuda()
    hidden = torch.randn(3, 8, 16, device="cuda")
    out, balance, dropped, overflow, domain = moe(hidden)
    flat = hidden.reshape(-1, 16).cpu().numpy()
    cap = moe.capacity(24)
    ref = oracle.moe_forward(flat, moe.router.weight.detach().cpu().numpy(), module_weights(moe), top_k=2, cap=cap,
                             dtype="f32")
    assert out.requires_grad  # parameters need grad: the differentiable path ran the same kernels
    assert np.allclose(out.detach().reshape(-1, 16).cpu().numpy(), ref["out"], atol=1e-5)
    assert int(overflow) == int(ref["plan"]["totals"][1]) == int(dropped)
    assert abs(float(balance.detach()) - ref["balance"]) < 1e-5
    assert out.shape == hidden.shape and balance.dtype == torch.float32 and overflow.dtype == torch.int64
    assert float(domain) == 0.0
    if capacity_factor:
        assert int(overflow) > 0


def test_capacity_keeps_highest_weight_routes_not_first_tokens():
    # tests/test_quantweave.py:116-127, observed through the plan instead of recorder experts
    cfg = qa.QuantaWeaveConfig(vocab_size=8, hidden_size=2, layers=1, ffn_size=2, num_experts=2, top_k=2,
                               attention_heads=1, max_sequence_length=4, capacity_factor=0.5, min_expert_capacity=1)
    moe = qa.TopKMoE(cfg).cuda()
    moe.router.weight.data = torch.tensor([[1.0, 0.0], [0.0, 0.0]], device="cuda")
    features = torch.tensor([0.5, 3.0, -2.0, 1.5])
    hidden = torch.stack([features, torch.zeros(4)], dim=-1)[None].cuda()
    _, _, dropped, overflow, _ = moe(hidden)
    assert overflow.item() == 4 and dropped.item() == 4
    kc = moe.last_plan["kept_counts"].tolist()
    assert kc == [2, 2]
    # kept tokens per expert: recover through the dropped list
    dt = moe.last_plan["dropped_token"][:4].tolist()
    de = moe.last_plan["dropped_expert"][:4].tolist()
    kept0 = sorted(features[t].item() for t in range(4) if (t, 0) not in zip(dt, de))
    kept1 = sorted(features[t].item() for t in range(4) if (t, 1) not in zip(dt, de))
    assert kept0 == [1.5, 3.0] and kept1 == [-2.0, 0.5]


def test_residual_policy_and_disabled_capacity():
    # tests/test_quantweave.py:129-147
    for overrides, exp_dropped, exp_overflow in ((dict(overflow_policy="residual"), 0, 4),
                                                 (dict(drop_overflow_tokens=False), 0, 0)):
        cfg = qa.QuantaWeaveConfig(vocab_size=8, hidden_size=2, layers=1, ffn_size=2, num_experts=2, top_k=2,
                                   attention_heads=1, max_sequence_length=4, capacity_factor=0.5,
                                   min_expert_capacity=1, **overrides)
        moe = qa.TopKMoE(cfg).cuda()
        moe.router.weight.data = torch.tensor([[1.0, 0.0], [0.0, 0.0]], device="cuda")
        hidden = torch.stack([torch.tensor([0.5, 3.0, -2.0, 1.5]), torch.zeros(4)], dim=-1)[None].cuda()
        _, _, dropped, overflow, _ = moe(hidden)
        assert dropped.item() == exp_dropped and overflow.item() == exp_overflow


def test_skipped_route_contributes_exactly_zero():
    # tests/test_quantweave.py:149-163
    cfg = qa.QuantaWeaveConfig(vocab_size=8, hidden_size=2, layers=1, ffn_size=4, num_experts=2, top_k=1,
                               attention_heads=1, max_sequence_length=4, capacity_factor=0.5, min_expert_capacity=1)
    moe = qa.TopKMoE(cfg).cuda()
    moe.router.weight.data = torch.tensor([[1.0, 0.0], [-1.0, 0.0]], device="cuda")
    hidden = torch.tensor([[[5.0, 1.0], [4.0, 1.0], [3.0, 1.0], [2.0, 1.0]]], device="cuda")
    output, _, _, overflow, _ = moe(hidden)
    assert overflow.item() == 3
    assert (output[0].abs().sum(-1) > 0).sum().item() == 1


def test_quantized_experts_take_the_grouped_path():
    torch.manual_seed(3)
    cfg = small_config(hidden_size=64, ffn_size=96, num_experts=8, attention_heads=1)
    moe = qa.TopKMoE(cfg).cuda()
    moe.to(torch.bfloat16)
    stats = qa.quantize_model(moe, 4)
    assert stats["replaced_layers"] == 8 * 3
    hidden = torch.randn(2, 40, 64, device="cuda").bfloat16()
    out, *_ = moe(hidden)
    w = dict(format="u4", d_model=64, d_ff=96, group_in=32, group_ff=32)
    for name in ("gate", "up", "down"):
        w[name] = np.stack([getattr(e, name).qweight.cpu().numpy() for e in moe.experts])
        w[name + "_scales"] = np.stack([getattr(e, name).scales.cpu().numpy() for e in moe.experts])
    flat = hidden.reshape(-1, 64).float().cpu().numpy()
    ref = oracle.moe_forward(flat, moe.router.weight.float().detach().cpu().numpy(), w, top_k=2, cap=moe.capacity(80),
                             dtype="bf16")
    assert normwise(out.reshape(-1, 64).float().cpu().numpy(), ref["out"]) <= 2e-2
    with pytest.raises(ValueError, match="already quantized"):
        qa.quantize_model(moe, 4)


def test_stats_and_static_dispatch():
    torch.manual_seed(1)
    moe = qa.TopKMoE(small_config(capacity_factor=0.5, min_expert_capacity=1)).cuda()
    moe.collect_stats = True
    hidden = torch.randn(2, 8, 16, device="cuda")
    _, _, dropped, overflow, _ = moe(hidden)
    st = moe.last_stats
    assert st["expert_load"].sum().item() == 32 - overflow.item()
    assert st["dropped_tokens"].numel() == overflow.item() == st["dropped_experts"].numel()
    assert st["expert_assigned"].sum().item() == 32
    moe.static_dispatch = True
    before = st
    _, _, dropped, overflow, _ = moe(hidden)
    assert overflow.item() == 0
    # the reference records stats on the dynamic path only (src/quantweave_moe_model.py:141-149)
    assert moe.last_stats is before


@pytest.mark.parametrize("T,E,k,cap", [(1, 64, 2, 2), (7, 8, 2, 3), (16, 64, 2, 32), (24, 6, 3, 5), (40, 16, 4, 4),
                                       (64, 64, 2, 128), (64, 8, 4, 20), (33, 1024, 2, 1), (3, 5, 5, 1)])
def test_small_batch_routing_and_plan_with_duplicate_tokens(T, E, k, cap):
    """Batches of up to 64 tokens are routed and planned in one workgroup; the
    result must equal the oracle's plan bit for bit, including equal weights
    (duplicated tokens: ordered by route id) and capacity drops."""
    w = W.Workload(f"small-T{T}-E{E}-k{k}", T, 256, E, 128, k, 1.0, "bf16", "bf16", 77 + T)
    layer = W.build_layer(w)
    if T > 2:
        layer.x[1::3] = layer.x[0]                 # every third token repeats token 0
    run = W.LayerRunner(layer, capacity=cap)
    run()
    torch.cuda.synchronize()
    logits = run.workspace_view("logits").cpu().numpy()
    probs_t = torch.softmax(run.workspace_view("logits"), dim=-1)
    assert torch.equal(run.probs, probs_t)
    res = oracle.moe_forward(layer.x.float().cpu().numpy(), layer.router.float().cpu().numpy(), host_weights(layer),
                             top_k=k, cap=cap, dtype="bf16", logits=logits, probs=probs_t.cpu().numpy())
    assert np.array_equal(run.top_idx.cpu().numpy(), res["top_idx"])
    assert np.array_equal(run.top_w.cpu().numpy().view(np.int32), res["top_w"].view(np.int32))
    assert np.array_equal(run.probs.cpu().numpy().view(np.int32), res["probs"].view(np.int32))
    p = res["plan"]
    kept, nd = int(p["totals"][0]), int(p["totals"][1])
    assert run.totals.cpu().tolist() == p["totals"].tolist()
    assert np.array_equal(run.counts.cpu().numpy(), p["counts"])
    assert np.array_equal(run.kept_counts.cpu().numpy(), p["kept_counts"])
    assert np.array_equal(run.workspace_view("kept_offsets").cpu().numpy(), p["kept_offsets"])
    assert np.array_equal(run.workspace_view("slot_token").cpu().numpy()[:kept], p["slot_token"])
    assert np.array_equal(run.workspace_view("slot_weight").cpu().numpy()[:kept].view(np.int32),
                          p["slot_weight"].view(np.int32))
    assert np.array_equal(run.workspace_view("route_slot").cpu().numpy(), p["route_slot"])
    assert np.array_equal(run.dropped_token.cpu().numpy()[:nd], p["dropped_token"])
    assert np.array_equal(run.dropped_expert.cpu().numpy()[:nd], p["dropped_expert"])
    assert normwise(run.out.float().cpu().numpy(), res["out"]) <= TOL["bf16"]


def test_layer_with_tiled_bf16_weights_is_identical():
    """The module packs bf16 experts into QW_BF16T tiles; the layer output is the
    same bit for bit as with the plain weights."""
    w = W.scaled(W.WORKLOADS["bf16-prefill-T8192-d2048-E64-f1024-k2"], tokens=1024, d_model=512, d_ff=256)
    layer = W.build_layer(w)
    plain = W.LayerRunner(layer)
    plain()
    tiled = W.LayerRunner(W.build_layer(w).add_tiles())
    assert "tiles" in tiled.layer.extra
    tiled()
    torch.cuda.synchronize()
    assert torch.equal(plain.out, tiled.out) and torch.equal(plain.top_idx, tiled.top_idx)


def test_expert_profiling_accumulates_time_per_expert():
    """tests/test_model_features.py:143-147: per-expert wall time with
    profile_experts, one timed call per expert with rows; the output is the
    layer's (to bf16 rounding: the experts run one launch each)."""
    torch.manual_seed(4)
    moe = qa.TopKMoE(small_config(hidden_size=64, ffn_size=128, num_experts=8, attention_heads=1)).cuda()
    hidden = torch.randn(2, 16, 64, device="cuda")
    with torch.no_grad():
        plain = moe(hidden)[0]
    moe.profile_experts = True
    out = moe(hidden)[0]
    assert sum(moe.expert_seconds) > 0
    used = moe.last_plan["kept_counts"].cpu()
    assert all((s > 0) == (c > 0) for s, c in zip(moe.expert_seconds, used.tolist()))
    assert normwise(out.detach().cpu().numpy(), plain.cpu().numpy()) <= 1e-4


def bf16_module(E=8, D=256, F_=512, k=2, cf=1.25, seed=5):
    cfg = small_config(hidden_size=D, ffn_size=F_, num_experts=E, top_k=k, attention_heads=1, capacity_factor=cf)
    torch.manual_seed(seed)
    return qa.TopKMoE(cfg).cuda().to(torch.bfloat16)


def bf16_module_weights(moe):
    w = dict(format="bf16", d_model=moe.router.in_features, d_ff=moe.experts[0].gate.out_features)
    for n in ("gate", "up", "down"):
        w[n] = np.stack([getattr(e, n).weight.detach().float().cpu().numpy() for e in moe.experts])
    return w


def test_loop_executor_selected_by_set_moe_kernel():
    """set_moe_kernel (src/quantweave_moe_model.py:381-393): "loop" launches one
    expert at a time, "triton"/"auto" all at once; both match the oracle, and
    the loop equals the grouped call to accumulation order."""
    moe = bf16_module()
    hidden = torch.randn(2, 160, 256, device="cuda").bfloat16()
    assert qa.set_moe_kernel(moe, "auto") == "triton" and moe.use_triton_kernels
    with torch.no_grad():
        grouped = moe(hidden)[0]
    assert qa.set_moe_kernel(moe, "loop") == "loop" and not moe.use_triton_kernels
    with torch.no_grad():
        looped, _, dropped, overflow, _ = moe(hidden)
    assert qa.set_moe_kernel(moe, "triton") == "triton" and qa.set_moe_kernel(moe, "hip") == "hip"
    flat = hidden.reshape(-1, 256).float().cpu().numpy()
    ref = oracle.moe_forward(flat, moe.router.weight.detach().float().cpu().numpy(), bf16_module_weights(moe), top_k=2,
                             cap=moe.capacity(320), dtype="bf16")
    for out in (grouped, looped):
        assert normwise(out.reshape(-1, 256).float().cpu().numpy(), ref["out"]) <= TOL["bf16"]
    assert int(overflow) == int(ref["plan"]["totals"][1])
    assert normwise(looped.float().cpu().numpy(), grouped.float().cpu().numpy()) <= 1e-2


def test_half_module_matches_oracle():
    """A TopKMoE in fp16 (`model.half()`): router, experts and hidden states in
    fp16; the experts packed into QW_F16T tiles; routing in fp32."""
    moe = bf16_module().half()
    hidden = torch.randn(2, 160, 256, device="cuda").half()
    with torch.no_grad():
        out, _, dropped, overflow, _ = moe(hidden)
    assert out.dtype == torch.float16
    from quantaweave_amd import _lib
    assert moe._qw_pack.fmt == _lib.QW_F16T
    flat = hidden.reshape(-1, 256).float().cpu().numpy()
    w = bf16_module_weights(moe)
    w["format"] = "f16"
    ref = oracle.moe_forward(flat, moe.router.weight.detach().float().cpu().numpy(), w, top_k=2,
                             cap=moe.capacity(320), dtype="f16")
    assert np.array_equal(moe.last_top_indices.cpu().numpy(), ref["top_idx"])
    assert int(overflow) == int(ref["plan"]["totals"][1])
    assert normwise(out.reshape(-1, 256).float().cpu().numpy(), ref["out"]) <= TOL["f16"]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_static_dispatch_matches_the_reference_static_output(dtype):
    """TopKMoE._static_output (src/quantweave_moe_model.py:235-245): capacity
    off, route weights cast to the hidden dtype before the product, a rounding
    per add; in fp32 it equals the dynamic path with capacity off
    (tests/test_model_features.py:49-56)."""
    moe = bf16_module(cf=0.5) if dtype == "bf16" else bf16_module(cf=0.5).float()
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    hidden = torch.randn(2, 96, 256, device="cuda").to(tdt)
    moe.static_dispatch = True
    with torch.no_grad():
        out, _, dropped, overflow, _ = moe(hidden)
    assert int(overflow) == 0 and int(dropped) == 0
    flat = hidden.reshape(-1, 256).float().cpu().numpy()
    w = bf16_module_weights(moe)
    w["format"] = dtype
    rw = moe.router.weight.detach().float().cpu().numpy()
    ref = oracle.moe_forward(flat, rw, w, top_k=2, cap=192 * 2, dtype=dtype)
    p = ref["plan"]
    static_ref = oracle.combine_static(ref["y"], p["slot_token"], p["slot_weight"], 192, dtype)
    got = out.reshape(-1, 256).float().cpu().numpy()
    assert normwise(got, static_ref) <= TOL[dtype]
    moe.static_dispatch = False
    moe.capacity_factor = 0.0
    with torch.no_grad():
        dynamic = moe(hidden)[0]
    if dtype == "f32":
        assert torch.equal(out, dynamic)
    else:  # only the bf16 cast of the route weights separates the two
        assert normwise(got, dynamic.reshape(-1, 256).float().cpu().numpy()) <= 1e-2


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("k", [2, 3, 4, 6, 12, 20])
def test_combine_is_bit_exact_against_the_oracle(k, dt):
    """qw_moe_combine_weighted from bf16 expert rows: torch's index_add_ rule
    (fp32 sum in plan order, one rounding) bit for bit, also at k >= 3 where a
    rounding per add would differ; and the static-dispatch combine.  Capacity
    1.0 drops 49 to 100 routes, so some tokens add fewer rows than k; k = 6,
    12 and 20 take the kernel's route bounds of 8, 16 and 64 (rows requested
    four at a time, and one at a time above 16)."""
    from quantaweave_amd import _hip, _lib

    T, D, E = 700, 512, (16 if k <= 16 else 24)
    g = torch.Generator().manual_seed(40 + k)
    _, idx, w = oracle.route_from_logits((torch.randn(T, E, generator=g) * 2).numpy(), k)
    p = oracle.plan(idx, w, E, oracle.capacity(T, k, E, 1.0))
    n = len(p["slot_token"])
    tdt, code = (torch.bfloat16, _lib.QW_BF16) if dt == "bf16" else (torch.float16, _lib.QW_F16)
    y = oracle.round_act((torch.randn(n, D, generator=g) * torch.logspace(-3, 3, D)[None]).numpy(), dt)
    yd = torch.from_numpy(y).cuda().to(tdt)
    slot = torch.from_numpy(p["route_slot"]).cuda()
    tidx = torch.from_numpy(idx).cuda()
    tw = torch.from_numpy(w).cuda()
    for fn, ref in (("qw_moe_combine_weighted", oracle.combine(y, p["slot_token"], p["slot_weight"], T, dt)),
                    ("qw_moe_combine_static", oracle.combine_static(y, p["slot_token"], p["slot_weight"], T, dt))):
        out = torch.empty(T, D, dtype=tdt, device="cuda")
        _lib.call(fn, _hip.ptr(yd), code, _hip.ptr(slot), _hip.ptr(tidx), _hip.ptr(tw), T, k, D, _hip.ptr(out),
                  code, _hip.stream(out.device))
        torch.cuda.synchronize()
        assert np.array_equal(out.float().cpu().numpy(), ref), fn


@pytest.mark.parametrize("T,E,K", [(8192, 64, 2), (100, 184, 3), (1, 8, 1), (4097, 1024, 4)])
def test_balance_with_workspace_matches_float64_and_is_deterministic(T, E, K):
    """qw_moe_balance_ws (per-64-token partial sums, fixed order) and
    qw_moe_balance: importance = probs.mean(0) and the balance term
    E * sum(importance * counts / (T*K)) (src/quantweave_moe_model.py:152-154)."""
    from quantaweave_amd import _hip, _lib

    g = torch.Generator().manual_seed(T + E)
    probs = torch.softmax(torch.randn(T, E, generator=g) * 3, dim=-1)
    counts = torch.randint(0, 2 * T * K // E + 2, (E,), generator=g, dtype=torch.int32)
    imp64 = probs.double().mean(0)
    bal64 = float(E * (imp64 * counts.double() / (T * K)).sum())
    pd, cd = probs.cuda(), counts.cuda()
    lib = _lib.load()
    nb = lib.qw_moe_balance_workspace_bytes(T, E)
    ws = _hip.workspace(nb, pd.device)
    outs = []
    for _ in range(2):
        imp = torch.empty(E, device="cuda")
        bal = torch.empty((), device="cuda")
        _lib.call("qw_moe_balance_ws", _hip.ptr(pd), _hip.ptr(cd), T, K, E, _hip.ptr(imp), _hip.ptr(bal),
                  _hip.ptr(ws), nb, _hip.stream(pd.device))
        outs.append((imp.cpu(), bal.cpu()))
    imp0 = torch.empty(E, device="cuda")
    bal0 = torch.empty((), device="cuda")
    _lib.call("qw_moe_balance", _hip.ptr(pd), _hip.ptr(cd), T, K, E, _hip.ptr(imp0), _hip.ptr(bal0),
              _hip.stream(pd.device))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    for imp, bal in (outs[0], (imp0.cpu(), bal0.cpu())):
        assert (imp.double() - imp64).abs().max() <= 1e-6 * max(imp64.abs().max().item(), 1e-30)
        assert abs(float(bal) - bal64) <= 1e-5 * max(abs(bal64), 1e-30)
    # the workspace form's fixed fp32 order, restated: bit for bit
    imp_ref, bal_ref = _balance_fixed_order(probs.numpy(), counts.numpy(), T, K, E)
    assert np.array_equal(outs[0][0].numpy(), imp_ref)
    assert outs[0][1].numpy().astype(np.float32) == bal_ref


def _balance_fixed_order(probs, counts, T, K, E):
    """qw_moe_balance_ws's additions in order, in float32: per 64-token chunk
    four strided sums (tokens j, j + 4, ... of the chunk) added as ((s0 + s1) + s2)
    + s3; 16 running sums over the chunk rows w, w + 16, ... (8 rows per step);
    those added in order; / T; terms imp * (count / (T K)) added in ascending
    expert order, times E."""
    f32 = np.float32
    nb = (T + 63) // 64
    partial = np.zeros((nb, E), f32)
    for b in range(nb):
        q = []
        for j in range(4):
            acc = np.zeros(E, f32)
            for i in range(16):
                t = 64 * b + j + 4 * i
                if t < min(T, 64 * b + 64):
                    acc = (acc + probs[t]).astype(f32)
            q.append(acc)
        partial[b] = (((q[0] + q[1]).astype(f32) + q[2]).astype(f32) + q[3]).astype(f32)
    tot = np.zeros(E, f32)
    for w in range(16):
        acc = np.zeros(E, f32)
        b0 = w
        while b0 < nb:
            for i in range(8):
                if b0 + 16 * i < nb:
                    acc = (acc + partial[b0 + 16 * i]).astype(f32)
            b0 += 128
        tot = (tot + acc).astype(f32)
    imp = (tot / f32(T)).astype(f32)
    term = (imp * (counts.astype(f32) / f32(T * K))).astype(f32)
    acc = f32(0)
    for e in range(E):
        acc = f32(acc + term[e])
    return imp, f32(f32(E) * acc)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_fast_decoder_prefill_composition(dt):
    """The call FastDecoder._prefill makes (src/fast_decode.py:219-235): fp32
    hidden states under bf16 (fp16) autocast, drop_overflow_tokens=False, and
    static_dispatch on (dense: E*n <= 4096) or off.  Each output is checked
    against the oracle on the run's routing (rows and weights rounded to the
    autocast type, expert arithmetic in that type, route terms added in fp32:
    index_add_ in plan order for the sorted path, the per-expert loop of
    _static_output for the dense one), and the two paths agree as in
    tests/test_fast_decode.py:70-79 (atol 1e-5)."""
    print(f"case prefill composition {dt}", flush=True)
    torch.manual_seed(21)
    moe = qa.TopKMoE(small_config(hidden_size=64, ffn_size=128, num_experts=8, capacity_factor=1.0)).cuda()
    n = 40
    x = torch.randn(n, 64, device="cuda")
    hidden = torch.nn.functional.layer_norm(x, (64,)).unsqueeze(0)           # [1, n, d] fp32
    name = "bf16" if dt == torch.bfloat16 else "f16"
    outs = {}
    for dense in (True, False):
        moe.drop_overflow_tokens, moe.static_dispatch = False, dense
        with torch.no_grad(), torch.autocast("cuda", dtype=dt):
            res = moe(hidden)
        out = res[0][0].float()
        assert res[0].dtype == torch.float32 and int(res[3]) == 0             # no capacity: nothing overflows
        plan = moe.last_plan
        top_idx = moe.last_top_indices.cpu().numpy().astype(np.int32)
        top_w = plan["top_w"].cpu().numpy()
        p = oracle.plan(top_idx, top_w, 8, n * 2)
        rows = oracle.round_act(hidden[0].cpu().numpy()[p["slot_token"]], name)
        y = oracle.experts_forward(rows, p["kept_counts"], module_weights(moe), name)
        combine = oracle.combine_static if dense else oracle.combine
        ref = combine(y, p["slot_token"], p["slot_weight"], n, "f32")
        err = normwise(out.cpu().numpy(), ref)
        print(f"  dense={dense} normwise {err:.3e}", flush=True)
        assert err <= TOL[name]
        outs[dense] = out
    moe.drop_overflow_tokens, moe.static_dispatch = True, False
    assert torch.allclose(outs[True], outs[False], atol=1e-5)
