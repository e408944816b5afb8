"""Grouped SwiGLU experts, grouped matmul and quantised linear on the GPU vs the oracle.

Tolerances (normwise, max|got-ref| / max|ref|): 1e-4 for fp32, 2e-2 for
bf16 / int8 / int4 weights with fp32 accumulation.
"""

import numpy as np
import pytest
import torch

import oracle
import quantaweave_amd as qa
from quantaweave_amd import _hip, _lib
from quantaweave_amd import moe_kernels as mk
from tests import hipcall as H

pytestmark = pytest.mark.gpu

COUNTS = [0, 5, 37, 1, 0, 64, 33, 2]          # empty experts, partial tiles, exact multiples (tests/test_moe_kernels.py:24)
TOL = {"f32": 1e-4, "bf16": 2e-2, "f16": 5e-3}
TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


# The streaming decode kernels against the reference's rounded-weight product
# (normwise): measured at most 9.05e-3 (bf16) and 7.8e-4 (fp16) over
# test_quantized_decode_rows_match_oracle's cases; bound with a margin, inside
# the layer tolerances TOL above: 2e-2 (bf16) and 5e-3 (fp16).
DECODE_DEV = {"bf16": 1.2e-2, "f16": 1.5e-3}
# Fractions of outputs equal to / within one ulp of the restatement of the
# kernels' own arithmetic: measured minima 0.959 / 0.987 (bf16) and
# 0.683 / 0.875 (fp16, int4's offset form), bounded a little below.
OWN_MATCH = {"bf16": (0.95, 0.98), "f16": (0.65, 0.85)}


def ulps16(got, ref, dtype):
    """Distance in units of the last place of the 16-bit type between two
    arrays of values representable in it."""
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    if dtype == "bf16":
        a = (got.view(np.uint32) >> 16).astype(np.int64)
        b = (ref.view(np.uint32) >> 16).astype(np.int64)
    else:
        a = got.astype(np.float16).view(np.uint16).astype(np.int64)
        b = ref.astype(np.float16).view(np.uint16).astype(np.int64)
    sign = 0x8000
    # ordered integer keys: negative values below positive ones
    ka = np.where(a & sign, -(a & (sign - 1)), a)
    kb = np.where(b & sign, -(b & (sign - 1)), b)
    return np.abs(ka - kb)


def normwise(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)


def make_weights(E, D, F_, fmt, seed, group=None, scale=0.05):
    rng = np.random.RandomState(seed)
    g32 = (rng.randn(E, F_, D) * scale).astype(np.float32)
    u32 = (rng.randn(E, F_, D) * scale).astype(np.float32)
    d32 = (rng.randn(E, D, F_) * scale).astype(np.float32)
    w = dict(format=fmt, d_model=D, d_ff=F_)
    if fmt in ("f32", "bf16", "f16"):
        w.update(gate=oracle.round_act(g32, fmt), up=oracle.round_act(u32, fmt), down=oracle.round_act(d32, fmt))
        return w
    bits = 8 if fmt == "i8" else 4
    for name, arr in (("gate", g32), ("up", u32), ("down", d32)):
        qs = [oracle.quantize(arr[e], bits, group) for e in range(E)]
        w[name] = np.stack([q for q, _, _ in qs])
        w[name + "_scales"] = np.stack([s for _, s, _ in qs])
        w["group_in" if name != "down" else "group_ff"] = qs[0][2]
    return w


def device_weights(w):
    fmt = w["format"]
    code = {"f32": _lib.QW_F32, "bf16": _lib.QW_BF16, "f16": _lib.QW_F16, "i8": _lib.QW_I8, "u4": _lib.QW_U4}[fmt]
    out = dict(fmt=code)
    for name in ("gate", "up", "down"):
        a = w[name]
        if fmt in ("bf16", "f16"):
            out[name] = H.dev(a, TORCH_DT[fmt])
        else:
            out[name] = H.dev(a)
        if fmt in ("i8", "u4"):
            out[name + "_s"] = H.dev(w[name + "_scales"])
    if fmt in ("i8", "u4"):
        out["group_in"], out["group_ff"] = w["group_in"], w["group_ff"]
    return out


def run_experts(x_np, counts, w, act, row_weight=None, row_index=None, x_rows=None, path="auto"):
    dw = device_weights(w)
    x = H.dev(x_np, TORCH_DT[act])
    offsets = H.dev(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32))
    y = H.experts(x, offsets, dw["fmt"], dw["gate"], dw["up"], dw["down"], dw.get("gate_s"), dw.get("up_s"),
                  dw.get("down_s"), dw.get("group_in", 0), dw.get("group_ff", 0),
                  row_index=None if row_index is None else H.dev(row_index.astype(np.int32)),
                  row_weight=None if row_weight is None else H.dev(row_weight.astype(np.float32)),
                  max_rows=int(sum(counts)), rows_per_expert=int(max(counts)), path=path)
    return y.float().cpu().numpy()


CASES = [
    ("f32", "f32", 48, 80, None), ("f32", "f32", 33, 17, None), ("bf16", "bf16", 64, 96, None),
    ("bf16", "bf16", 256, 512, None), ("bf16", "i8", 64, 96, None), ("bf16", "i8", 40, 24, 16),
    ("bf16", "u4", 64, 96, None), ("bf16", "u4", 40, 24, 16), ("f32", "i8", 64, 64, None), ("f32", "u4", 64, 64, 32),
    ("f16", "f16", 64, 96, None), ("f16", "f16", 256, 512, None), ("f16", "i8", 64, 96, None),
    ("f16", "u4", 40, 24, 16), ("f16", "f32", 48, 80, None), ("f16", "bf16", 64, 96, None),
    ("bf16", "f16", 64, 96, None), ("f32", "f16", 48, 80, None),
]


@pytest.mark.parametrize("path", ["auto", "generic"])
@pytest.mark.parametrize("act,fmt,D,F_,group", CASES)
def test_grouped_swiglu_matches_oracle(act, fmt, D, F_, group, path):
    print(f"case act={act} fmt={fmt} D={D} F={F_} group={group} path={path}", flush=True)
    rng = np.random.RandomState(D + F_)
    rows = sum(COUNTS)
    x = rng.randn(rows, D).astype(np.float32)
    x = oracle.round_act(x, act)
    w = make_weights(len(COUNTS), D, F_, fmt, D * F_, group)
    rw = rng.rand(rows).astype(np.float32)
    got = run_experts(x, COUNTS, w, act, row_weight=rw, path=path)
    ref = oracle.round_act(oracle.experts_forward(x, np.array(COUNTS), w, act) * rw[:, None], act)
    assert np.isfinite(got).all()
    assert normwise(got, ref) <= TOL[act]


@pytest.mark.parametrize("E,D,F_,rows", [(16, 1024, 256, 100), (8, 256, 512, 128), (2, 2048, 256, 1000),
                                         (3, 256, 512, 128), (2, 64, 96, 60), (5, 256, 128, 100)])
def test_fp32_tile_sizes_match_oracle(E, D, F_, rows):
    """fp32 experts on the matrix cores: enough 64 x 64 down tiles to fill the GPU
    (the 64 x 64 kernel) and a small layer (32 x 32 tiles, K split over the waves).
    The kernels walk (column tile, expert, row chunk) in XCD order: with fewer
    than 8 experts an expert spans 8 // E XCDs (2 and 3 experts), and with 5
    experts three XCDs get no work; every tile must still be visited once."""
    print(f"case f32 E={E} D={D} F={F_} rows~{rows}", flush=True)
    rng = np.random.RandomState(E + D)
    counts = [int(c) for c in rng.randint(rows - 40, rows + 40, size=E)]
    counts[1] = 0
    n = sum(counts)
    x = rng.randn(n, D).astype(np.float32)
    w = make_weights(E, D, F_, "f32", D + F_)
    rw = rng.rand(n).astype(np.float32)
    got = run_experts(x, counts, w, "f32", row_weight=rw)
    ref = oracle.experts_forward(x, np.array(counts), w, "f32") * rw[:, None]
    assert np.isfinite(got).all()
    assert normwise(got, ref) <= TOL["f32"]


@pytest.mark.parametrize("act,fmt,group,path", [
    ("bf16", "bf16", None, "mfma"), ("bf16", "bf16", None, "stream"), ("bf16", "bf16", None, "generic"),
    ("bf16", "i8", None, "stream"), ("bf16", "i8", None, "generic"), ("bf16", "u4", 32, "stream"),
    ("bf16", "u4", 32, "generic"), ("f32", "f32", None, "generic"), ("f32", "f32", None, "mfma"),
    ("bf16", "i8", None, "mfma"), ("bf16", "i8", 64, "mfma"), ("bf16", "u4", 32, "mfma"), ("bf16", "u4", 128, "mfma"),
    ("f16", "f16", None, "mfma"), ("f16", "f16", None, "stream"), ("f16", "f16", None, "generic"),
    ("f16", "i8", None, "mfma"), ("f16", "u4", 32, "mfma"), ("f16", "i8", None, "stream"), ("f16", "u4", 32, "stream")])
def test_each_kernel_family_matches_oracle(act, fmt, group, path):
    """The same inputs through every kernel family that takes them
    (qw_moe_experts_on_path), each against the oracle."""
    print(f"case family act={act} fmt={fmt} path={path}", flush=True)
    D, F_ = 256, 512
    rng = np.random.RandomState(17)
    rows = sum(COUNTS)
    x = oracle.round_act(rng.randn(rows, D).astype(np.float32), act)
    w = make_weights(len(COUNTS), D, F_, fmt, 23, group)
    rw = rng.rand(rows).astype(np.float32)
    got = run_experts(x, COUNTS, w, act, row_weight=rw, path=path)
    ref = oracle.round_act(oracle.experts_forward(x, np.array(COUNTS), w, act) * rw[:, None], act)
    assert normwise(got, ref) <= TOL[act]


@pytest.mark.parametrize("act,fmt,group,D,F_", [
    ("bf16", "u4", 32, 512, 1408),    # gate/up 16 chunks per row (1 slot, whole), down 44 (3 slots, clamped)
    ("bf16", "u4", 32, 1024, 3072),   # 2 slots whole; down 96 chunks (6 slots, whole)
    ("bf16", "u4", 32, 2048, 4096),   # 4 slots whole; down 128 chunks (8 slots, whole)
    ("bf16", "u4", 32, 1536, 2560),   # 3 slots whole; down 80 chunks (6 slots, clamped)
    ("bf16", "u4", 64, 1024, 1408),   # two chunks per scale (not whole)
    ("bf16", "u4", 128, 4096, 1024),  # 8 slots, four chunks per scale
    ("f16", "u4", 32, 4096, 1408),    # the int4 decode layer's rows with fp16 activations
    ("bf16", "u4", 32, 6144, 512),    # gate/up rows of 192 chunks take the dot-product kernel
    ("bf16", "u4", 2048, 2048, 2048),  # one scale per row: 4 slots in two row sets, loaded once per row set
    ("bf16", "i8", None, 2048, 1024),  # the int8 decode layer: one scale per row, 8 and 4 slots
    ("bf16", "i8", 16, 256, 512),     # one scale per chunk, whole rows (1 and 2 slots)
    ("bf16", "i8", 16, 2048, 1024),   # one scale per chunk, whole rows of 8 and 4 slots: scale blocks
    ("bf16", "i8", 64, 1536, 768),    # 6 slots, four chunks per scale; down 3 slots
    ("f16", "i8", None, 2048, 1024),  # fp16 activations (used unscaled)
    ("bf16", "i8", None, 4096, 1024),  # gate/up rows of 256 chunks take the dot-product kernel
])
def test_quantized_decode_rows_match_oracle(act, fmt, group, D, F_):
    """int4 / int8 experts at decode row counts (1 to 9 rows, so one to three
    passes of 4 routes) through the weight-streaming family, whose quantised rows
    of up to 128 chunks run on the 4x4x4 matrix-core kernel.

    Two checks.  (1) Against a restatement of the kernels' own arithmetic
    (exact codes times fp32 group scales, sums in float64, the SwiGLU's 16-bit
    rounding points): most outputs are the same 16-bit value and nearly all
    within one ulp (OWN_MATCH; what differs is fp32 summation order, and with
    fp16 activations the offset form 1024 + u of the codes, whose correction
    term cancels in fp32) — a wrong scale or offset on any chunk moves whole
    rows and fails this.  (2) Against the reference's arithmetic, which rounds
    each q * scale to the activation type before the product
    (src/quantization.py:71-72): the streaming kernels skip that rounding
    (only ~37% of outputs are then the same value), and the deviation measured
    over these cases, with a margin, bounds the comparison (DECODE_DEV)."""
    print(f"case quantised decode act={act} fmt={fmt} group={group} D={D} F={F_}", flush=True)
    _check_quantized_decode(act, fmt, group, D, F_, [1, 0, 3, 9, 2])


@pytest.mark.parametrize("act,fmt,group,D,F_", [
    ("bf16", "u4", 32, 4096, 1408),   # the int4 decode layer's shapes
    ("bf16", "i8", None, 2048, 1024),  # the int8 decode layer's shapes
])
def test_quantized_decode_many_passes(act, fmt, group, D, F_):
    """Experts with 5 to 17 routes at decode sizes: each pass of up to 4 routes
    is its own column of blocks (14 passes over 6 experts here, an empty expert
    among them), checked as test_quantized_decode_rows_match_oracle."""
    print(f"case quantised decode passes act={act} fmt={fmt} D={D} F={F_}", flush=True)
    _check_quantized_decode(act, fmt, group, D, F_, [17, 0, 5, 13, 1, 8])


def _check_quantized_decode(act, fmt, group, D, F_, counts):
    rng = np.random.RandomState(D + F_ + (group or 0))
    rows = sum(counts)
    x = oracle.round_act(rng.randn(rows, D).astype(np.float32), act)
    w = make_weights(len(counts), D, F_, fmt, D * 7 + F_, group)
    rw = rng.rand(rows).astype(np.float32)
    got = run_experts(x, counts, w, act, row_weight=rw, path="stream")
    assert np.isfinite(got).all()
    own = oracle.round_act(oracle.experts_forward(x, np.array(counts), w, act, quantised="exact") * rw[:, None], act)
    ulps = ulps16(got, own, act)
    own_nw = normwise(got, own)
    ref = oracle.round_act(oracle.experts_forward(x, np.array(counts), w, act) * rw[:, None], act)
    dev = normwise(got, ref)
    print(f"  own arithmetic: normwise {own_nw:.3e}, {np.mean(ulps == 0):.4f} equal, {np.mean(ulps <= 1):.5f} "
          f"within 1 ulp; reference rounding: normwise {dev:.3e}, {np.mean(ulps16(got, ref, act) == 0):.4f} equal",
          flush=True)
    equal, within = OWN_MATCH[act]
    assert np.mean(ulps == 0) >= equal and np.mean(ulps <= 1) >= within
    assert dev <= DECODE_DEV[act]


def test_kernel_family_that_does_not_take_the_format_refuses():
    # the matrix-core kernels take quantisation groups of whole 32-column K steps
    w = make_weights(len(COUNTS), 256, 512, "i8", 3, group=16)
    x = oracle.round_bf16(np.random.RandomState(0).randn(sum(COUNTS), 256).astype(np.float32))
    with pytest.raises(RuntimeError, match="matrix-core"):
        run_experts(x, COUNTS, w, "bf16", path="mfma")


@pytest.mark.parametrize("act,fmt,group,D,F_,counts", [
    ("bf16", "i8", None, 512, 256, [300, 0, 17, 64, 320, 1]), ("bf16", "i8", 64, 512, 256, [300, 0, 17, 64, 320, 1]),
    ("bf16", "u4", 32, 512, 256, [300, 0, 17, 64, 320, 1]), ("bf16", "u4", 128, 256, 512, [40, 200, 3]),
    ("bf16", "i8", None, 2048, 1024, [256, 250, 262, 241]), ("bf16", "u4", 32, 2048, 1024, [256, 250, 262, 241]),
    ("f16", "i8", None, 512, 256, [300, 0, 17, 64, 320, 1]), ("f16", "u4", 32, 2048, 1024, [256, 250, 262, 241])])
def test_quantised_mfma_equals_bf16_mfma_of_dequantised_weights(act, fmt, group, D, F_, counts):
    """The matrix-core path dequantises each weight to bf16(q * scale), the
    reference's dequantize().to(bfloat16) (src/quantization.py:61-72), and then
    runs the bf16 kernel's MFMA sequence: its outputs equal, bit for bit, those
    of the bf16 path given the dequantised weights.  The same for fp16."""
    print(f"case quantised mfma act={act} fmt={fmt} group={group} D={D} F={F_} counts={counts}", flush=True)
    rng = np.random.RandomState(D + len(counts))
    rows = sum(counts)
    x = oracle.round_act(rng.randn(rows, D).astype(np.float32), act)
    w = make_weights(len(counts), D, F_, fmt, 5, group)
    deq = dict(format=act, d_model=D, d_ff=F_)
    for name, gname in (("gate", "group_in"), ("up", "group_in"), ("down", "group_ff")):
        cols = F_ if name == "down" else D
        deq[name] = oracle.round_act(np.stack([
            oracle.dequantize(w[name][e], w[name + "_scales"][e], 8 if fmt == "i8" else 4, cols, w[gname])
            for e in range(len(counts))]), act)
    rw = rng.rand(rows).astype(np.float32)
    got = run_experts(x, counts, w, act, row_weight=rw, path="mfma")
    ref = run_experts(x, counts, deq, act, row_weight=rw, path="mfma")
    assert np.array_equal(got.view(np.int32), ref.view(np.int32))


def test_gathered_rows_through_row_index():
    rng = np.random.RandomState(0)
    D, F_ = 64, 128
    x_all = oracle.round_bf16(rng.randn(50, D).astype(np.float32))
    counts = [3, 0, 20, 9]
    row_index = rng.randint(0, 50, size=sum(counts)).astype(np.int32)
    w = make_weights(4, D, F_, "bf16", 1)
    got = run_experts(x_all, counts, w, "bf16", row_index=row_index)
    ref = oracle.experts_forward(x_all[row_index], np.array(counts), w, "bf16")
    assert normwise(got, ref) <= 2e-2


@pytest.mark.parametrize("in_features,out_features", [(48, 80), (64, 64), (33, 17)])
def test_grouped_matmul_matches_per_expert_matmuls(in_features, out_features):
    # tests/test_moe_kernels.py:27-36 (forward)
    torch.manual_seed(0)
    x = torch.randn(sum(COUNTS), in_features, device="cuda")
    weight = torch.randn(len(COUNTS), out_features, in_features, device="cuda")
    plan = mk.GroupedPlan(COUNTS, x.device)
    y = mk.grouped_matmul(x, weight, plan)
    parts, start = [], 0
    for e, c in enumerate(COUNTS):
        parts.append(x[start:start + c].double() @ weight[e].double().t())
        start += c
    expected = torch.cat(parts).float()
    assert torch.allclose(y, expected, atol=1e-4, rtol=1e-4)


def test_grouped_matmul_bf16_is_close_and_all_empty_plan_is_safe():
    # tests/test_moe_kernels.py:50-59
    torch.manual_seed(1)
    x = torch.randn(sum(COUNTS), 64, device="cuda", dtype=torch.bfloat16)
    weight = torch.randn(len(COUNTS), 96, 64, device="cuda", dtype=torch.bfloat16)
    y = mk.grouped_matmul(x, weight, mk.GroupedPlan(COUNTS, x.device))
    parts, start = [], 0
    for e, c in enumerate(COUNTS):
        parts.append(x[start:start + c].double() @ weight[e].double().t())
        start += c
    expected = torch.cat(parts)
    assert (y.double() - expected).abs().max() < 0.25 and y.dtype == torch.bfloat16
    empty = mk.grouped_matmul(torch.empty(0, 64, device="cuda"), weight.float(), mk.GroupedPlan([0] * len(COUNTS), x.device))
    assert empty.shape == (0, 96)


@pytest.mark.parametrize("in_features", [128, 40])
def test_grouped_matmul_f16_matches_per_expert_matmuls(in_features):
    """fp16 operands: the matrix-core GEMM (in_features % 64 == 0) or the
    general kernel, fp32 accumulation, one rounding to fp16."""
    torch.manual_seed(3)
    x = torch.randn(sum(COUNTS), in_features, device="cuda").half()
    weight = (torch.randn(len(COUNTS), 96, in_features, device="cuda") * 0.1).half()
    y = mk.grouped_matmul(x, weight, mk.GroupedPlan(COUNTS, x.device))
    assert y.dtype == torch.float16
    parts, start = [], 0
    for e, c in enumerate(COUNTS):
        parts.append(x[start:start + c].double() @ weight[e].double().t())
        start += c
    expected = torch.cat(parts)
    assert normwise(y.double().cpu().numpy(), expected.cpu().numpy()) <= 2e-3


def test_grouped_swiglu_api_matches_oracle_over_real_experts():
    # tests/test_moe_kernels.py:62-84 (forward)
    torch.manual_seed(2)
    config = qa.QuantaWeaveConfig(vocab_size=8, hidden_size=48, layers=1, ffn_size=72, num_experts=len(COUNTS), top_k=1,
                                  attention_heads=1, max_sequence_length=8)
    moe = qa.TopKMoE(config).cuda()
    x = torch.randn(sum(COUNTS), 48, device="cuda")
    with torch.no_grad():
        fused = mk.grouped_swiglu(x, moe.experts, COUNTS)  # fused gate/up + down kernels
    composed = mk.grouped_swiglu(x, moe.experts, COUNTS)  # differentiable composition (weights need grad)
    assert composed.requires_grad and not fused.requires_grad
    w = dict(format="f32", d_model=48, d_ff=72,
             gate=np.stack([e.gate.weight.detach().cpu().numpy() for e in moe.experts]),
             up=np.stack([e.up.weight.detach().cpu().numpy() for e in moe.experts]),
             down=np.stack([e.down.weight.detach().cpu().numpy() for e in moe.experts]))
    ref = oracle.experts_forward(x.cpu().numpy(), np.array(COUNTS), w, "f32")
    for out in (fused, composed):
        assert np.allclose(out.detach().cpu().numpy(), ref, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("bits,group,shape", [(8, None, (24, 40)), (4, 16, (24, 40)), (4, None, (1408, 4096)),
                                              (8, None, (1024, 2048)), (4, 8, (5, 8))])
def test_quantized_linear_bytes_match_oracle(bits, group, shape):
    torch.manual_seed(bits)
    lin = torch.nn.Linear(shape[1], shape[0], bias=False)
    lin.weight.data.mul_(0.5)
    q = qa.QuantizedLinear.from_linear(lin.cuda(), bits, group)
    oq, os_, og = oracle.quantize(lin.weight.detach().cpu().numpy(), bits, group)
    assert np.array_equal(q.qweight.cpu().numpy(), oq)
    assert np.array_equal(q.scales.cpu().numpy(), os_)
    deq = q.dequantize().cpu().numpy()
    assert np.array_equal(deq, oracle.dequantize(oq, os_, bits, shape[1], og))


def test_int4_lossless_known_answer_on_gpu():
    # tests/test_deploy_and_distill.py:173-184
    lin = torch.nn.Linear(8, 1, bias=False)
    lin.weight.data = torch.tensor([[-7, -1, 0, 1, 7, 3, -4, 2]], dtype=torch.float32) * 0.5
    q = qa.QuantizedLinear.from_linear(lin.cuda(), 4, 8)
    assert q.scales.item() == 0.5
    assert torch.equal(q.dequantize(), lin.weight.detach())


@pytest.mark.parametrize("bits,group,max_rel", [(8, None, 0.02), (4, 16, 0.2)])
def test_quantized_linear_forward(bits, group, max_rel):
    # tests/test_deploy_and_distill.py:161-171 plus oracle parity of the forward itself
    torch.manual_seed(0)
    lin = torch.nn.Linear(40, 24, bias=False).cuda()
    q = qa.QuantizedLinear.from_linear(lin, bits, group)
    for dtype, tol in ((torch.float32, 1e-5), (torch.bfloat16, 2e-2), (torch.float16, 5e-3)):
        name = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dtype]
        x = torch.randn(5, 40, device="cuda").to(dtype)
        got = q(x).float().cpu().numpy()
        assert q(x).dtype == dtype
        deq = oracle.round_act(q.dequantize().cpu().numpy(), name)
        ref = oracle.linear(x.float().cpu().numpy(), deq, name)
        assert normwise(got, ref) <= tol
        err = np.linalg.norm(got - (x.float() @ lin.weight.T).detach().cpu().numpy()) / np.linalg.norm(ref)
        assert err < max_rel + (0.02 if dtype != torch.float32 else 0)
    assert q.stored_bytes() < lin.weight.numel() * 4 / (3.5 if bits == 8 else 4)


# ---------------------------------------------------------------- QW_BF16T tiled weights
def test_bf16_tile_packing_matches_the_layout():
    rng = np.random.RandomState(70)
    w = oracle.round_bf16(rng.randn(3, 48, 128).astype(np.float32))
    tiled = qa.moe.tile_bf16(H.dev(w, torch.bfloat16))
    torch.cuda.synchronize()
    assert np.array_equal(tiled.float().cpu().numpy(), oracle.tile_bf16(w))
    with pytest.raises(ValueError, match="64"):
        bad = H.dev(np.zeros((1, 8, 32), np.float32), torch.bfloat16)
        _lib.call("qw_pack_bf16_tiles", H.P(bad), 1, 8, 32, H.P(torch.empty_like(bad)), H.s())


@pytest.mark.parametrize("counts,D,F_", [
    ([40, 0, 70, 33, 64, 1], 128, 256),   # prefill-sized rows: MFMA kernels
    ([1, 0, 3, 2], 256, 512),             # decode-sized rows: weight-streaming kernels
    ([1, 0, 2], 4096, 128),               # decode-sized rows longer than the streaming kernel takes: general kernel
])
def test_tiled_bf16_weights_give_identical_outputs(counts, D, F_):
    """The tiles change where each weight is read, not the arithmetic: the
    outputs equal those from the plain layout bit for bit, on every path."""
    print(f"case tiles counts={counts} D={D} F={F_}", flush=True)
    rng = np.random.RandomState(D + F_ + 1)
    rows = sum(counts)
    x = oracle.round_bf16(rng.randn(rows, D).astype(np.float32))
    w = make_weights(len(counts), D, F_, "bf16", D * F_ + 3)
    rw = rng.rand(rows).astype(np.float32)
    plain = run_experts(x, counts, w, "bf16", row_weight=rw)
    dw = device_weights(w)
    offsets = H.dev(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32))
    tiled = H.experts(H.dev(x, torch.bfloat16), offsets, _lib.QW_BF16T, qa.moe.tile_bf16(dw["gate"]),
                      qa.moe.tile_bf16(dw["up"]), qa.moe.tile_bf16(dw["down"]),
                      row_weight=H.dev(rw), max_rows=rows, rows_per_expert=max(counts)).float().cpu().numpy()
    assert np.array_equal(plain, tiled)
    ref = oracle.round_act(oracle.experts_forward(x, np.array(counts), w, "bf16") * rw[:, None], "bf16")
    assert normwise(tiled, ref) <= 2e-2


def test_tiled_bf16_shape_errors():
    x = H.dev(np.zeros((4, 48), np.float32), torch.bfloat16)
    wt = H.dev(np.zeros((1, 64, 48), np.float32), torch.bfloat16)
    wd = H.dev(np.zeros((1, 48, 64), np.float32), torch.bfloat16)
    offsets = H.dev(np.array([0, 4], np.int32))
    with pytest.raises(ValueError, match="multiples of 64"):
        H.experts(x, offsets, _lib.QW_BF16T, wt, wt, wd, max_rows=4, rows_per_expert=4)


@pytest.mark.parametrize("N,K", [(64, 48), (18, 48)])
def test_grouped_matmul_f32_output_offset_by_one_float(N, K):
    """The fp32 matrix-core kernel stores 16-byte vectors; an output view that
    starts one float into a buffer (or rows of N % 4 != 0 floats) must take
    the general kernel and give the same values."""
    print(f"case grouped matmul f32 offset N={N} K={K}", flush=True)
    torch.manual_seed(4)
    counts = [5, 0, 12, 3]
    rows = sum(counts)
    x = torch.randn(rows, K, device="cuda")
    w = torch.randn(len(counts), N, K, device="cuda")
    offsets = H.dev(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32))

    def run(out):
        _lib.call("qw_grouped_matmul", H.P(x), _lib.QW_F32, H.P(w), _lib.QW_F32, None, 0, len(counts), N, K,
                  H.P(offsets), rows, max(counts), H.P(out), H.s())
        torch.cuda.synchronize()
        return out.clone()

    aligned = run(torch.empty(rows, N, device="cuda"))
    buf = torch.full((rows * N + 1,), float("nan"), device="cuda")
    shifted = run(buf[1:].view(rows, N))
    assert torch.isnan(buf[0])
    ref = torch.cat([x[s:s + c].double() @ w[e].double().t()
                     for e, (s, c) in enumerate(zip(np.cumsum([0] + counts[:-1]), counts))])
    assert torch.allclose(aligned.double(), ref, atol=1e-4, rtol=1e-4)
    assert torch.allclose(shifted.double(), ref, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("D", [2048, 4096])
def test_int8_decode_route_of_tiny_activations(D):
    """int8 rows with bf16 activations scale each route by a power of two so
    its values are exact in fp16; a route whose largest |x| is below 2^-112
    must not overflow that scale (its output is ~0, not NaN).  D=2048 runs the
    matrix-core kernel, D=4096 the dot-product one."""
    print(f"case int8 decode tiny route D={D}", flush=True)
    counts = [2, 3]
    rng = np.random.RandomState(D)
    x = rng.randn(sum(counts), D).astype(np.float32)
    x[1] *= 2.0 ** -120
    x[3] *= 2.0 ** -126
    x = oracle.round_bf16(x)
    w = make_weights(len(counts), D, 1024, "i8", 11)
    got = run_experts(x, counts, w, "bf16", path="stream")
    assert np.isfinite(got).all()
    ref = oracle.experts_forward(x, np.array(counts), w, "bf16")
    assert np.abs(got[[1, 3]]).max() <= 1e-30
    assert normwise(got, ref) <= DECODE_DEV["bf16"]


def test_prefill_hidden_rows_follow_the_reference_rounding():
    """The 16-bit prefill kernel forms silu with the hardware reciprocal
    (silu_fast).  Given the kernel's own gate and up projections (saved,
    already rounded to bf16), its hidden rows must equal the reference's
    rounding chain bf16(bf16(silu(g)) * u), silu computed in float64 and
    rounded to fp32 first as torch's fp32 opmath does: a value may differ only
    where silu(g) lies within a few fp32 ulp of a bf16 rounding boundary, so
    by at most one bf16 ulp and rarely (src/moe_kernels.py:194)."""
    print("case prefill hidden rows: silu rounding", flush=True)
    counts = [40, 64, 17, 100]
    E, D, F_ = len(counts), 256, 384
    rng = np.random.RandomState(7)
    rows = sum(counts)
    x = H.dev(rng.randn(rows, D).astype(np.float32), torch.bfloat16)
    w = [H.dev((rng.randn(E, a, b) * 0.06).astype(np.float32), torch.bfloat16) for a, b in ((F_, D), (F_, D), (D, F_))]
    offsets = H.dev(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32))
    outs = [torch.empty(rows, n, dtype=torch.bfloat16, device="cuda") for n in (D, F_, F_, F_, D)]
    y, g_out, u_out, h_out, y_unw = outs
    nb = _lib.load().qw_moe_experts_workspace_bytes(rows, E, D, F_, _lib.QW_BF16)
    ws = _hip.workspace(nb, torch.device("cuda"))
    P = _hip.ptr
    _lib.call("qw_moe_experts_save", P(x), _lib.QW_BF16, None, P(offsets), E, D, F_, rows, max(counts), _lib.QW_BF16,
              0, 0, P(w[0]), None, P(w[1]), None, P(w[2]), None, None, P(y), P(g_out), P(u_out), P(h_out), P(y_unw),
              P(ws), nb, H.s())
    torch.cuda.synchronize()
    g = g_out.double().cpu()
    u = u_out.double().cpu()
    silu = (g / (1.0 + torch.exp(-g))).float().bfloat16().double()
    want = (silu * u).float().bfloat16()
    got = h_out.cpu()
    ulps = (got.view(torch.int16).int() - want.view(torch.int16).int()).abs().numpy()
    equal = float(np.mean(ulps == 0))
    print(f"  {ulps.size} hidden values: {equal:.6f} equal, max {int(ulps.max())} ulp", flush=True)
    assert int(ulps.max()) <= 1 and equal >= 0.999
