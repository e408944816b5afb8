"""The torch-CPU restatement of the reference's forward (oracle/torch_ref.py,
the CPU baseline of bench.py) against the numpy/C oracle: two independent
restatements of src/quantweave_moe_model.py:113-211 and
src/quantization.py:61-72 must agree — routing and plan exactly, outputs to
accumulation order."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import torch_ref


def make(fmt, E=8, D=64, F_=96, seed=0, group=None):
    g = torch.Generator().manual_seed(seed)
    w32 = [torch.randn(E, F_, D, generator=g) * 0.05, torch.randn(E, F_, D, generator=g) * 0.05,
           torch.randn(E, D, F_, generator=g) * 0.05]
    host = dict(format=fmt, d_model=D, d_ff=F_)
    if fmt in ("f32", "bf16"):
        dt = torch.float32 if fmt == "f32" else torch.bfloat16
        ws = [w.to(dt) for w in w32]
        for n, w in zip(("gate", "up", "down"), ws):
            host[n] = w.float().numpy()
        return torch_ref.Experts(fmt, *ws), host
    bits = 8 if fmt == "i8" else 4
    stacks, scales = [], []
    for n, w in zip(("gate", "up", "down"), w32):
        qs = [oracle.quantize(w[e].numpy(), bits, group) for e in range(E)]
        host[n] = np.stack([q for q, _, _ in qs])
        host[n + "_scales"] = np.stack([s for _, s, _ in qs])
        host["group_ff" if n == "down" else "group_in"] = qs[0][2]
        stacks.append(torch.from_numpy(host[n]))
        scales.append(torch.from_numpy(host[n + "_scales"]))
    return torch_ref.Experts(fmt, *stacks, *scales), host


@pytest.mark.parametrize("fmt,act,cf,k", [("f32", "f32", 1.25, 2), ("f32", "f32", 0.6, 3), ("bf16", "bf16", 1.0, 2),
                                          ("i8", "bf16", 0.0, 2), ("u4", "bf16", 0.0, 2), ("u4", "f32", 1.25, 1)])
def test_torch_restatement_equals_the_oracle(fmt, act, cf, k):
    T, D, E = 300, 64, 8
    experts, host = make(fmt, E=E, D=D, group=32 if fmt == "u4" else None)
    g = torch.Generator().manual_seed(7)
    dt = torch.float32 if act == "f32" else torch.bfloat16
    x = torch.randn(T, D, generator=g).to(dt)
    router = (torch.randn(E, D, generator=g) * 0.3).to(dt)
    cap = oracle.capacity(T, k, E, cf)
    out, balance, overflow, top_idx, kept_counts = torch_ref.moe_forward(x, router, experts, k, cap)
    logits = F.linear(x.float(), router.float()).numpy()
    ref = oracle.moe_forward(x.float().numpy(), router.float().numpy(), host, top_k=k, cap=cap, dtype=act,
                             logits=logits)
    assert np.array_equal(top_idx.numpy(), ref["top_idx"])
    assert np.array_equal(kept_counts.numpy(), ref["plan"]["kept_counts"])
    assert overflow == int(ref["plan"]["totals"][1])
    got, want = out.float().numpy(), ref["out"]
    tol = 1e-5 if act == "f32" else 2e-2
    assert np.abs(got - want).max() <= tol * np.abs(want).max()
    assert abs(float(balance) - ref["balance"]) < 1e-5
    if cf and cf < 1.25:
        assert overflow > 0


def test_dequantize_matches_the_oracle_bytes():
    w = torch.randn(24, 64) * 0.05
    for bits, group in ((8, None), (4, 32), (4, 16)):
        q, s, grp = oracle.quantize(w.numpy(), bits, group)
        got = torch_ref.dequantize(torch.from_numpy(q), torch.from_numpy(s), bits, 64)
        assert np.array_equal(got.numpy(), oracle.dequantize(q, s, bits, 64, grp))
