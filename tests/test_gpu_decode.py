"""One-token MoE decode step (qw_moe_decode_step / MoEDecodeStep) against the oracle.

The step is the routed-expert part of FastDecoder._step (src/fast_decode.py:170-177):
fp32 routing with selection on the scores, no capacity, experts in their
stored format, fp32 weighted sum added to the residual.  Routing is compared
bit for bit given the kernel's scores; the MoE output normwise within 1e-4
(fp32) or 2e-2 (bf16 / int8 / int4); HIP-graph replays bit for bit against
eager calls.
"""

import numpy as np
import pytest
import torch

import oracle
import quantaweave_amd as qa
from quantaweave_amd import _lib

pytestmark = pytest.mark.gpu

TOL = {"fp32": 1e-4, "bf16": 2e-2, "fp16": 5e-3}


def normwise(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)


def make_moe(E, D, F_, k, fmt, seed, temperature=1.0, bias=False, group=None):
    cfg = qa.QuantaWeaveConfig(vocab_size=8, hidden_size=D, layers=1, ffn_size=F_, num_experts=E, top_k=k,
                               attention_heads=1, max_sequence_length=4, capacity_factor=0,
                               router_temperature=temperature)
    torch.manual_seed(seed)
    moe = qa.TopKMoE(cfg)
    with torch.no_grad():
        moe.router.weight.normal_(0, 0.05)
        for e in moe.experts:
            for p in (e.gate, e.up, e.down):
                p.weight.normal_(0, 0.05)
    moe = moe.cuda()
    if fmt == "bf16":
        moe.to(torch.bfloat16)
    elif fmt == "f16":
        moe.half()
    elif fmt in ("i8", "u4"):
        qa.quantize_model(moe, 8 if fmt == "i8" else 4, group)
    if bias:
        moe.expert_bias = torch.randn(E, generator=torch.Generator().manual_seed(seed + 1)).cuda()
    return moe


def oracle_weights(step):
    """The expert weights the step multiplies, as the oracle's weight dict."""
    p = step.pack
    fmt = {_lib.QW_F32: "f32", _lib.QW_BF16: "bf16", _lib.QW_BF16T: "bf16", _lib.QW_F16: "f16",
           _lib.QW_F16T: "f16", _lib.QW_I8: "i8", _lib.QW_U4: "u4"}[p.fmt]
    w = dict(format=fmt, d_model=step.hidden, d_ff=step.ffn, group_in=p.group_in, group_ff=p.group_ff)
    for name in ("gate", "up", "down"):
        t = getattr(p, name)
        w[name] = t.float().cpu().numpy() if fmt in ("f32", "bf16", "f16") else t.cpu().numpy()
        if p.fmt in (_lib.QW_BF16T, _lib.QW_F16T):
            w[name] = oracle.untile_bf16(w[name])
        s = getattr(p, name + "_s")
        if s is not None:
            w[name + "_scales"] = s.cpu().numpy()
    return w


def check_step(moe, T, precision, seed=7):
    E, D = moe.router.weight.shape
    print(f"case decode T={T} d={D} E={E} f={moe.experts[0].gate.out_features} k={moe.top_k} {precision}",
          flush=True)
    step = qa.MoEDecodeStep(moe, precision=precision, tokens=T)
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(T, D, device="cuda", generator=g)
    resid = torch.randn(T, D, device="cuda", generator=g)
    moe_only = step(x).clone()
    scores = step.scores().cpu().numpy()
    out = step(x, resid).clone()
    torch.cuda.synchronize()
    xs = x.cpu().numpy()
    rw = step.router.cpu().numpy()
    ref_scores = oracle.router_logits(xs, rw, step.temperature)
    assert np.abs(scores - ref_scores).max() <= 1e-5 * max(1.0, np.abs(ref_scores).max())
    bias = None if step.bias is None else step.bias.cpu().numpy()
    dtype = {"fp32": "f32", "bf16": "bf16", "fp16": "f16"}[precision]
    probs_t = torch.softmax(step.scores(), dim=-1)             # torch's softmax on this device
    assert torch.equal(step.probs, probs_t)
    res = oracle.decode_step(xs, rw, oracle_weights(step), top_k=step.top_k, dtype=dtype,
                             temperature=step.temperature, expert_bias=bias, logits=scores,
                             probs=probs_t.cpu().numpy())
    # bit-exact routing given the scores
    assert np.array_equal(step.probs.cpu().numpy().view(np.int32), res["probs"].view(np.int32))
    assert np.array_equal(step.last_top_indices.cpu().numpy(), res["top_idx"])
    assert np.array_equal(step.last_top_weights.cpu().numpy().view(np.int32), res["top_w"].view(np.int32))
    got = moe_only.cpu().numpy()
    assert np.isfinite(got).all()
    assert normwise(got, res["out"]) <= TOL[precision]
    # the residual is added last, in fp32
    assert torch.equal(out, resid + moe_only)
    return step, x, resid


CASES = [
    # (E, D, F, k, fmt, group, T, precision)
    (8, 256, 384, 2, "f32", None, 1, "fp32"),
    (8, 256, 384, 2, "f32", None, 3, "bf16"),
    (16, 512, 256, 2, "bf16", None, 1, "bf16"),
    (16, 512, 256, 4, "bf16", None, 5, "bf16"),
    (16, 512, 256, 6, "bf16", None, 2, "bf16"),   # the combine's bound of 8 routes
    (16, 512, 256, 10, "i8", None, 1, "bf16"),    # above 8 routes: the combine's per-route loop
    (16, 512, 256, 2, "i8", None, 1, "bf16"),
    (16, 512, 256, 2, "i8", None, 2, "fp32"),
    (16, 1024, 352, 2, "u4", 32, 1, "bf16"),
    (16, 1024, 352, 3, "u4", 32, 4, "bf16"),
    (8, 96, 40, 2, "u4", 8, 1, "bf16"),
    (16, 512, 256, 2, "f16", None, 1, "fp16"),
    (16, 512, 256, 4, "f16", None, 5, "fp16"),
    (8, 256, 384, 2, "f32", None, 3, "fp16"),
    (16, 512, 256, 2, "bf16", None, 2, "fp16"),
    (16, 512, 256, 2, "i8", None, 1, "fp16"),
    (16, 1024, 352, 3, "u4", 32, 4, "fp16"),
]


@pytest.mark.parametrize("E,D,F_,k,fmt,group,T,precision", CASES)
def test_decode_step_matches_oracle(E, D, F_, k, fmt, group, T, precision):
    check_step(make_moe(E, D, F_, k, fmt, seed=E + D + T, group=group), T, precision)


@pytest.mark.parametrize("precision", ["bf16", "fp16"])
@pytest.mark.parametrize("fmt,D,F_,group", [("u4", 4096, 1408, 32), ("i8", 2048, 1024, None),
                                            ("bf16", 2048, 1024, None)])
def test_decode_step_full_size(fmt, D, F_, group, precision):
    """Batch-1 decode at the decode workloads' layer shapes (64 experts, top-2)."""
    check_step(make_moe(64, D, F_, 2, fmt, seed=3, group=group), 1, precision)


@pytest.mark.parametrize("top_k,temperature,bias", [(1, 1.0, False), (2, 1.0, False), (2, 0.7, True), (3, 2.0, False)])
def test_decode_step_reproduces_the_layer_forward(top_k, temperature, bias):
    """tests/test_fast_decode.py:40-56 at the MoE block: the step equals the
    layer forward with capacity off, in fp32, to 1e-5."""
    moe = make_moe(8, 32, 48, top_k, "f32", seed=top_k, temperature=temperature, bias=bias)
    moe.drop_overflow_tokens = False
    step = qa.MoEDecodeStep(moe, precision="fp32", tokens=6)
    x = torch.randn(6, 32, device="cuda", generator=torch.Generator(device="cuda").manual_seed(5))
    resid = torch.randn(6, 32, device="cuda", generator=torch.Generator(device="cuda").manual_seed(6))
    got = step(x, resid)
    full, *_ = moe(x[None])
    torch.cuda.synchronize()
    assert torch.equal(step.last_top_indices.long(), moe.last_top_indices.long())
    assert torch.allclose(got, resid + full[0], atol=1e-5)


def test_in_place_residual_and_bias_steering():
    moe = make_moe(8, 256, 128, 2, "bf16", seed=11)
    step = qa.MoEDecodeStep(moe, tokens=2)
    x = torch.randn(2, 256, device="cuda")
    resid = torch.randn(2, 256, device="cuda")
    expected = resid + step(x)
    step(x, resid, out=resid)
    assert torch.equal(resid, expected)
    # tests/test_parallelism.py:345-357: a bias of -100 keeps an expert out
    moe.expert_bias = torch.zeros(8, device="cuda")
    moe.expert_bias[3] = -100.0
    biased = qa.MoEDecodeStep(moe, tokens=2)
    for _ in range(3):
        biased(torch.randn(2, 256, device="cuda") * 10)
        assert not (biased.last_top_indices == 3).any()


def test_quantized_step_keeps_packed_bytes():
    moe = make_moe(8, 256, 128, 2, "u4", seed=12, group=32)
    step = qa.MoEDecodeStep(moe)
    assert step.pack.gate.dtype == torch.uint8 and step.pack.gate.shape == (8, 128, 128)
    assert step.pack.down.shape == (8, 256, 64)


def test_graph_replays_match_eager_calls():
    """The step recorded in a HIP graph (as FastDecoder records its step,
    src/fast_decode.py:178-204) gives the eager result on every replay."""
    moe = make_moe(64, 1024, 352, 2, "u4", seed=13, group=32)
    step = qa.MoEDecodeStep(moe, tokens=1)
    x_static = torch.zeros(1, 1024, device="cuda")
    r_static = torch.zeros(1, 1024, device="cuda")
    out_static = torch.zeros(1, 1024, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step(x_static, r_static, out_static)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(x_static, r_static, out_static)
    g = torch.Generator(device="cuda").manual_seed(14)
    for i in range(5):
        x = torch.randn(1, 1024, device="cuda", generator=g)
        r = torch.randn(1, 1024, device="cuda", generator=g)
        x_static.copy_(x)
        r_static.copy_(r)
        graph.replay()
        torch.cuda.synchronize()
        replayed = out_static.clone()
        idx_replayed = step.last_top_indices.clone()
        eager = step(x, r).clone()
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), i
        assert torch.equal(idx_replayed, step.last_top_indices), i
