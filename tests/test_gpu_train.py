"""Backward pass on the GPU: grouped matmul, grouped SwiGLU and the MoE layer
against the float64 autograd oracle (oracle/train.py).

Restates tests/test_moe_kernels.py:29-57 (grouped matmul forward/backward:
outputs and input gradients atol 1e-4, weight gradients atol 1e-3, exact-zero
weight gradients for experts without rows, bf16 and an all-empty plan),
:60-82 (grouped_swiglu gradients vs the per-expert loop, atol 1e-3) and
:86-105 (the layer's output and gradients, capacity off and on, atol 1e-3),
with the float64 oracle in place of the reference's loop path.
"""

import numpy as np
import pytest
import torch

import quantaweave_amd as qa
from oracle import train as tr
from quantaweave_amd import moe_kernels as mk

pytestmark = pytest.mark.gpu

COUNTS = [0, 5, 37, 1, 0, 64, 33, 2]


def cpu64(t):
    return t.detach().double().cpu()


def normwise(got, want):
    want = want.detach().double()
    return ((cpu64(got).reshape(want.shape) - want).abs().max() / want.abs().max().clamp_min(1e-30)).item()


@pytest.mark.parametrize("in_features,out_features", [(48, 80), (64, 64), (33, 17)])
def test_grouped_matmul_forward_and_backward(in_features, out_features):
    print(f"case grouped_matmul {in_features}x{out_features}", flush=True)
    torch.manual_seed(0)
    x = torch.randn(sum(COUNTS), in_features, device="cuda", requires_grad=True)
    weight = torch.randn(len(COUNTS), out_features, in_features, device="cuda", requires_grad=True)
    plan = mk.GroupedPlan(COUNTS, x.device)
    y = mk.grouped_matmul(x, weight, plan)
    upstream = torch.randn_like(y)
    y.backward(upstream)
    xr = cpu64(x).requires_grad_()
    wr = cpu64(weight).requires_grad_()
    ref = tr.grouped_matmul(xr, wr, COUNTS)
    ref.backward(cpu64(upstream))
    assert torch.allclose(cpu64(y), ref.detach(), atol=1e-4, rtol=1e-4)
    assert torch.allclose(cpu64(x.grad), xr.grad, atol=1e-4, rtol=1e-4)
    assert torch.allclose(cpu64(weight.grad), wr.grad, atol=1e-3, rtol=1e-4)
    for e, count in enumerate(COUNTS):
        if count == 0:
            assert weight.grad[e].abs().sum() == 0  # experts with no rows get an exactly-zero gradient


def test_grouped_matmul_bf16_backward_and_empty_plan():
    print("case grouped_matmul bf16", flush=True)
    torch.manual_seed(1)
    x = torch.randn(sum(COUNTS), 64, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    weight = torch.randn(len(COUNTS), 96, 64, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    y = mk.grouped_matmul(x, weight, mk.GroupedPlan(COUNTS, x.device))
    assert y.dtype == torch.bfloat16
    upstream = torch.randn_like(y)
    y.backward(upstream)
    assert x.grad.dtype == torch.bfloat16 and weight.grad.dtype == torch.bfloat16
    xr, wr = cpu64(x).requires_grad_(), cpu64(weight).requires_grad_()
    ref = tr.grouped_matmul(xr, wr, COUNTS)
    ref.backward(cpu64(upstream))
    assert (cpu64(y) - ref.detach()).abs().max() < 0.25
    for got, want in ((x.grad, xr.grad), (weight.grad, wr.grad)):
        err = (cpu64(got) - want).abs().max() / want.abs().max()
        assert err < 2e-2
    # all-empty plan: empty output, zero weight gradient, empty input gradient
    xe = torch.empty(0, 64, device="cuda", requires_grad=True)
    we = weight.detach().float().requires_grad_()
    empty = mk.grouped_matmul(xe, we, mk.GroupedPlan([0] * len(COUNTS), xe.device))
    assert empty.shape == (0, 96)
    empty.sum().backward()
    assert xe.grad.shape == (0, 64) and (we.grad == 0).all()


def make_moe(E, D, F_, K, capacity_factor=0.0, seed=0):
    config = qa.QuantaWeaveConfig(vocab_size=8, hidden_size=D, layers=1, ffn_size=F_, num_experts=E, top_k=K,
                                  attention_heads=1, max_sequence_length=512, capacity_factor=capacity_factor,
                                  min_expert_capacity=1)
    torch.manual_seed(seed)
    return qa.TopKMoE(config).cuda()


def stacks(moe):
    return [torch.stack([getattr(e, n).weight.detach() for e in moe.experts]).double().cpu()
            for n in ("gate", "up", "down")]


def test_grouped_swiglu_gradients_match_the_per_expert_loop():
    print("case grouped_swiglu 48x72", flush=True)
    moe = make_moe(len(COUNTS), 48, 72, 1, seed=2)
    x = torch.randn(sum(COUNTS), 48, device="cuda", requires_grad=True)
    out = mk.grouped_swiglu(x, moe.experts, COUNTS)
    out.square().sum().backward()
    xr = cpu64(x).requires_grad_()
    ws = [w.requires_grad_() for w in stacks(moe)]
    ref = tr.grouped_swiglu(xr, *ws, COUNTS)
    ref.square().sum().backward()
    assert torch.allclose(cpu64(out), ref.detach(), atol=1e-4, rtol=1e-4)
    assert torch.allclose(cpu64(x.grad), xr.grad, atol=1e-3, rtol=1e-3)
    for name, w in zip(("gate", "up", "down"), ws):
        got = torch.stack([getattr(e, name).weight.grad for e in moe.experts])
        assert torch.allclose(cpu64(got), w.grad, atol=1e-3, rtol=1e-3), name
    for e, count in enumerate(COUNTS):
        if count == 0:
            assert moe.experts[e].gate.weight.grad.abs().sum() == 0


def test_grouped_swiglu_under_bf16_autocast():
    print("case grouped_swiglu autocast", flush=True)
    moe = make_moe(len(COUNTS), 64, 128, 1, seed=5)
    x = torch.randn(sum(COUNTS), 64, device="cuda", requires_grad=True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = mk.grouped_swiglu(x, moe.experts, COUNTS)
    assert out.dtype == torch.bfloat16
    out.float().square().sum().backward()
    assert x.grad.dtype == torch.float32 and moe.experts[0].gate.weight.grad.dtype == torch.float32
    xr = cpu64(x).requires_grad_()
    ws = [w.requires_grad_() for w in stacks(moe)]
    ref = tr.grouped_swiglu(xr, *ws, COUNTS)
    ref.square().sum().backward()
    err = (cpu64(x.grad) - xr.grad).abs().max() / xr.grad.abs().max()
    assert err < 3e-2
    got = torch.stack([e.down.weight.grad for e in moe.experts])
    assert (cpu64(got) - ws[2].grad).abs().max() / ws[2].grad.abs().max() < 3e-2


def layer_reference(moe, x, domains=None):
    """The oracle's layer forward on the run's own routing, with gradients."""
    plan = moe.last_plan
    top_idx = moe.last_top_indices.cpu()
    n_drop = int(plan["totals"][1])
    kept = tr.kept_routes(top_idx, plan["dropped_token"].cpu().long(), plan["dropped_expert"].cpu().long(), n_drop)
    xr = cpu64(x).reshape(-1, x.size(-1)).requires_grad_()
    rw = cpu64(moe.router.weight).requires_grad_()
    ws = [w.requires_grad_() for w in stacks(moe)]
    out, probs, balance = tr.moe_layer(xr, rw, *ws, top_idx, kept, moe.router_temperature)
    return out, probs, balance, xr, rw, ws, n_drop


@pytest.mark.parametrize("capacity_factor", [0.0, 0.7])
def test_layer_output_and_gradients(capacity_factor):
    print(f"case layer grads cf={capacity_factor}", flush=True)
    moe = make_moe(16, 64, 96, 2, capacity_factor, seed=3)
    x = torch.randn(4, 96, 64, device="cuda", requires_grad=True)
    out, balance, dropped, overflow, _ = moe(x)
    (out.square().sum() + balance).backward()
    ref, probs, bal, xr, rw, ws, n_drop = layer_reference(moe, x)
    (ref.square().sum() + bal).backward()
    assert overflow.item() == n_drop
    if capacity_factor:
        assert n_drop > 0  # the run exercised dropped routes
    assert torch.allclose(cpu64(out).reshape(ref.shape), ref.detach(), atol=1e-4, rtol=1e-4)
    assert abs(balance.item() - bal.item()) < 1e-5
    assert torch.allclose(cpu64(x.grad).reshape(xr.shape), xr.grad, atol=1e-3, rtol=1e-3)
    assert torch.allclose(cpu64(moe.router.weight.grad), rw.grad, atol=1e-3, rtol=1e-3)
    for name, w in zip(("gate", "up", "down"), ws):
        got = torch.stack([getattr(e, name).weight.grad for e in moe.experts])
        assert torch.allclose(cpu64(got), w.grad, atol=1e-3, rtol=1e-3), name
        assert normwise(got, w.grad) <= 1e-4, name
    assert normwise(x.grad, xr.grad) <= 1e-4
    assert normwise(moe.router.weight.grad, rw.grad) <= 1e-4


def test_layer_gradients_with_bias_temperature_and_domain_loss():
    print("case layer grads bias/temperature/domains", flush=True)
    moe = make_moe(8, 64, 64, 3, 1.0, seed=6)
    moe.router_temperature = 0.7
    moe.expert_bias = torch.linspace(-0.5, 0.5, 8, device="cuda")
    x = torch.randn(2, 40, 64, device="cuda", requires_grad=True)
    domains = torch.randint(0, 3, (2, 40), device="cuda", generator=torch.Generator(device="cuda").manual_seed(1))
    out, balance, _, _, domain_loss = moe(x, domains, 3)
    (out.square().mean() + 0.1 * balance + domain_loss).backward()
    ref, probs, bal, xr, rw, ws, _ = layer_reference(moe, x)
    # the domain loss of the reference (src/quantweave_moe_model.py:247-257) on the oracle's probabilities
    member = torch.nn.functional.one_hot(domains.reshape(-1).cpu(), 3).double()
    counts = member.sum(0)
    prof = torch.nn.functional.normalize((member.t() @ probs) / counts.clamp(min=1)[:, None], dim=-1)
    prof = prof[counts > 0]
    sim = prof @ prof.t()
    dl = (sim.sum() - sim.diagonal().sum()) / (prof.size(0) * (prof.size(0) - 1))
    assert abs(domain_loss.item() - dl.item()) < 1e-5
    (ref.square().mean() + 0.1 * bal + dl).backward()
    assert normwise(x.grad, xr.grad) <= 1e-4
    assert normwise(moe.router.weight.grad, rw.grad) <= 1e-4
    for name, w in zip(("gate", "up", "down"), ws):
        assert normwise(torch.stack([getattr(e, name).weight.grad for e in moe.experts]), w.grad) <= 1e-4, name


def test_layer_bf16_gradients_within_tolerance():
    print("case layer grads bf16", flush=True)
    moe = make_moe(16, 128, 256, 2, 1.25, seed=7).to(torch.bfloat16)
    x = torch.randn(2, 64, 128, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    out, balance, *_ = moe(x)
    (out.float().square().sum() + balance).backward()
    ref, probs, bal, xr, rw, ws, _ = layer_reference(moe, x)
    (ref.square().sum() + bal).backward()
    assert x.grad.dtype == torch.bfloat16
    for got, want in ((x.grad.reshape(xr.shape), xr.grad), (moe.router.weight.grad, rw.grad),
                      (torch.stack([e.gate.weight.grad for e in moe.experts]), ws[0].grad)):
        assert (cpu64(got) - want).abs().max() / want.abs().max() < 3e-2


def test_layer_output_is_the_inference_output():
    """With autograd on, the forward runs the same kernels as under no_grad."""
    print("case layer train/inference forward", flush=True)
    moe = make_moe(16, 64, 96, 2, 1.0, seed=8)
    x = torch.randn(3, 50, 64, device="cuda")
    train_out = moe(x.clone().requires_grad_())[0]
    with torch.no_grad():
        infer_out = moe(x)[0]
    assert torch.equal(train_out.detach(), infer_out)


@pytest.mark.parametrize("E,D,F_,tokens,cf", [(16, 256, 512, 512, 1.25), (64, 256, 512, 16, 0.0)],
                         ids=["matrix-core", "weight-streaming"])
def test_bf16_layer_output_is_the_inference_output(E, D, F_, tokens, cf):
    """bf16 experts: the forward with autograd on (qw_moe_experts_save, which
    also keeps the activations) gives the inference call's output bit for bit,
    at a shape the matrix-core kernels take (64 rows per expert) and at one
    the weight-streaming kernels take (half a row per expert)."""
    print(f"case layer train/inference bf16 E={E} D={D} F={F_} T={tokens}", flush=True)
    moe = make_moe(E, D, F_, 2, cf, seed=12).to(torch.bfloat16)
    x = torch.randn(1, tokens, D, device="cuda").to(torch.bfloat16)
    train_out = moe(x.clone().requires_grad_())[0]
    with torch.no_grad():
        infer_out = moe(x)[0]
    assert torch.equal(train_out.detach(), infer_out)
    train_out.float().square().sum().backward()
    assert all(torch.isfinite(p.grad).all() for p in moe.parameters() if p.grad is not None)


def test_training_steps_reduce_the_loss():
    print("case layer sgd", flush=True)
    moe = make_moe(8, 64, 128, 2, 1.25, seed=9)
    g = torch.Generator(device="cuda").manual_seed(10)
    x = torch.randn(4, 32, 64, device="cuda", generator=g)
    target = torch.randn(4, 32, 64, device="cuda", generator=g) * 0.1
    opt = torch.optim.SGD(moe.parameters(), lr=0.5)
    losses = []
    for _ in range(8):
        opt.zero_grad()
        out, balance, *_ = moe(x)
        loss = (out - target).square().mean() + 0.01 * balance
        loss.backward()
        assert all(torch.isfinite(p.grad).all() for p in moe.parameters() if p.grad is not None)
        opt.step()
        losses.append(loss.item())
    assert losses[-1] < losses[0]


def test_layer_under_bf16_autocast():
    """Experts in bf16 on an fp32 stream: routing on the fp32 input, expert rows
    in bf16, (y * w) added in fp32 (src/quantweave_moe_model.py:126-127, :201;
    src/moe_kernels.py:179-195); forward equal with and without autograd."""
    print("case layer autocast", flush=True)
    moe = make_moe(16, 128, 256, 2, 1.25, seed=11)
    x = torch.randn(2, 64, 128, device="cuda", requires_grad=True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out, balance, *_ = moe(x)
    assert out.dtype == torch.float32
    (out.square().sum() + balance).backward()
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        infer = moe(x)[0]
    assert torch.equal(infer, out.detach())
    ref, probs, bal, xr, rw, ws, _ = layer_reference(moe, x)
    (ref.square().sum() + bal).backward()
    assert normwise(out, ref) <= 2e-2
    assert x.grad.dtype == torch.float32
    for got, want in ((x.grad, xr.grad), (moe.router.weight.grad, rw.grad),
                      (torch.stack([e.down.weight.grad for e in moe.experts]), ws[2].grad)):
        assert normwise(got, want) <= 3e-2


def test_layer_under_f16_autocast():
    """The same under fp16 autocast (the reference's --precision fp16 training,
    src/train_quantweave_moe.py:598-600): expert rows and weights in fp16,
    routing and the weighted sum in fp32."""
    print("case layer f16 autocast", flush=True)
    moe = make_moe(16, 128, 256, 2, 1.25, seed=13)
    x = torch.randn(2, 64, 128, device="cuda", requires_grad=True)
    with torch.autocast("cuda", dtype=torch.float16):
        out, balance, *_ = moe(x)
    assert out.dtype == torch.float32
    (out.square().sum() + balance).backward()
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
        infer = moe(x)[0]
    assert torch.equal(infer, out.detach())
    ref, probs, bal, xr, rw, ws, _ = layer_reference(moe, x)
    (ref.square().sum() + bal).backward()
    assert normwise(out, ref) <= 5e-3
    assert x.grad.dtype == torch.float32
    for got, want in ((x.grad, xr.grad), (moe.router.weight.grad, rw.grad),
                      (torch.stack([e.down.weight.grad for e in moe.experts]), ws[2].grad)):
        assert normwise(got, want) <= 1e-2


def test_grouped_swiglu_under_f16_autocast():
    print("case grouped_swiglu f16 autocast", flush=True)
    moe = make_moe(len(COUNTS), 64, 128, 1, seed=6)
    x = torch.randn(sum(COUNTS), 64, device="cuda", requires_grad=True)
    with torch.autocast("cuda", dtype=torch.float16):
        out = mk.grouped_swiglu(x, moe.experts, COUNTS)
    assert out.dtype == torch.float16
    out.float().square().sum().backward()
    xr = cpu64(x).requires_grad_()
    ws = [w.requires_grad_() for w in stacks(moe)]
    ref = tr.grouped_swiglu(xr, *ws, COUNTS)
    ref.square().sum().backward()
    assert (cpu64(out) - ref.detach()).abs().max() / ref.detach().abs().max() < 5e-3
    err = (cpu64(x.grad) - xr.grad).abs().max() / xr.grad.abs().max()
    assert err < 1e-2


def test_kernel_benchmark_reports_both_paths():
    # tests/test_moe_kernels.py:131-134: the reference's keys and checks
    result = mk.benchmark(experts=16, tokens=2048, hidden=64, ffn=128, repeats=3)
    assert result["loop_ms"] > 0 and result["triton_ms"] > 0 and result["speedup"] > 0
    assert result["speedup"] == result["loop_ms"] / result["triton_ms"] and result["forward_ms"] > 0
    result = mk.benchmark(experts=16, tokens=2048, hidden=64, ffn=128, repeats=2, bf16=True)
    assert result["loop_ms"] > 0 and result["triton_ms"] > 0 and result["bf16"]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("counts,in_features,out_features", [
    ([0, 5, 300, 1, 0, 129, 64, 2], 128, 192),     # matrix cores for dX (192 % 64 == 0) and dW
    ([7, 0, 200, 33], 320, 96),                    # dX on the vector ALUs (96 % 64 != 0), dW on the matrix cores
    ([1000, 24], 64, 2048),                        # many row tiles, many column tiles
])
def test_grouped_matmul_half_matrix_core_paths(counts, in_features, out_features, dtype):
    print(f"case grouped_matmul {dtype} {counts} {in_features}x{out_features}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(sum(counts))
    x = torch.randn(sum(counts), in_features, device="cuda", generator=g).to(dtype).requires_grad_()
    weight = (torch.randn(len(counts), out_features, in_features, device="cuda", generator=g) * 0.1).to(dtype)
    weight.requires_grad_()
    y = mk.grouped_matmul(x, weight, mk.GroupedPlan(counts, x.device))
    assert y.dtype == dtype
    upstream = torch.randn(y.shape, device="cuda", generator=g).to(dtype)
    y.backward(upstream)
    xr, wr = cpu64(x).requires_grad_(), cpu64(weight).requires_grad_()
    ref = tr.grouped_matmul(xr, wr, counts)
    ref.backward(cpu64(upstream))
    assert normwise(y, ref) <= 1e-2
    assert normwise(x.grad, xr.grad) <= 1e-2
    assert normwise(weight.grad, wr.grad) <= 1e-2
    for e, c in enumerate(counts):
        if c == 0:
            assert (weight.grad[e] == 0).all()
        else:  # every expert's gradient block is its own (no cross-expert mixing)
            assert normwise(weight.grad[e], wr.grad[e]) <= 1e-2
