"""Pins of the gradient oracle (oracle/train.py) on the CPU.

* Its layer forward equals the forward oracle (oracle.moe_forward, pinned
  against the reference's own tests elsewhere) given the same routing, with
  and without capacity drops — a dropped renormalisation, a wrong gather or a
  kept/dropped mix-up fails here.
* Its gradients match central finite differences (torch.autograd.gradcheck)
  with routing held fixed.
* The grouped matmul's gradients match their closed forms, dX = dY W_e and
  dW_e = dY_e^T X_e, and an expert without rows gets an exactly zero dW
  (tests/test_moe_kernels.py:29-47).
"""

import numpy as np
import pytest
import torch

import oracle
from oracle import train as tr

COUNTS = [0, 5, 37, 1, 0, 64, 33, 2]


def random_layer(T, D, F_, E, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, D, generator=g, dtype=torch.float64)
    rw = torch.randn(E, D, generator=g, dtype=torch.float64) * 0.5
    gate = torch.randn(E, F_, D, generator=g, dtype=torch.float64) * 0.2
    up = torch.randn(E, F_, D, generator=g, dtype=torch.float64) * 0.2
    down = torch.randn(E, D, F_, generator=g, dtype=torch.float64) * 0.2
    return x, rw, gate, up, down


@pytest.mark.parametrize("cf", [0.0, 0.7])
def test_layer_forward_equals_the_forward_oracle(cf):
    T, D, F_, E, K = 96, 16, 24, 8, 2
    x, rw, gate, up, down = random_layer(T, D, F_, E, seed=1)
    x32 = x.float().numpy()
    rw32 = rw.float().numpy()
    cap = oracle.capacity(T, K, E, cf, 1.0, 1, True)
    w = dict(format="f32", d_model=D, d_ff=F_, group_in=0, group_ff=0, gate=gate.float().numpy(),
             up=up.float().numpy(), down=down.float().numpy())
    ref = oracle.moe_forward(x32, rw32, w, top_k=K, cap=cap, dtype="f32")
    p = ref["plan"]
    top_idx = torch.from_numpy(ref["top_idx"].astype(np.int64))
    kept = tr.kept_routes(top_idx, torch.from_numpy(p["dropped_token"]), torch.from_numpy(p["dropped_expert"]),
                          int(p["totals"][1]))
    if cf:
        assert not kept.all()
    out, probs, balance = tr.moe_layer(x.float().double(), rw.float().double(), gate.float().double(),
                                       up.float().double(), down.float().double(), top_idx, kept)
    assert np.allclose(probs.numpy(), ref["probs"], rtol=1e-6, atol=1e-7)
    assert np.allclose(out.numpy(), ref["out"], rtol=1e-5, atol=1e-6)
    assert abs(balance.item() - ref["balance"]) <= 1e-6 * abs(ref["balance"])


def test_layer_gradients_match_finite_differences():
    T, D, F_, E, K = 6, 4, 3, 4, 2
    x, rw, gate, up, down = random_layer(T, D, F_, E, seed=2)
    with torch.no_grad():
        probs = (x @ rw.t()).softmax(-1)
    top_idx = probs.topk(K, dim=-1).indices
    kept = torch.ones(T, K, dtype=torch.bool)
    kept[1, 1] = False  # one dropped route

    def f(x, rw, gate, up, down):
        out, probs, balance = tr.moe_layer(x, rw, gate, up, down, top_idx, kept, temperature=0.8)
        return out, probs, balance

    inputs = tuple(t.clone().requires_grad_() for t in (x, rw, gate, up, down))
    assert torch.autograd.gradcheck(f, inputs, eps=1e-6, atol=1e-6, rtol=1e-5)


def test_grouped_matmul_gradients_have_their_closed_forms():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(sum(COUNTS), 33, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(len(COUNTS), 17, 33, generator=g, dtype=torch.float64, requires_grad=True)
    y = tr.grouped_matmul(x, w, COUNTS)
    dy = torch.randn(y.shape, generator=g, dtype=torch.float64)
    y.backward(dy)
    start = 0
    for e, c in enumerate(COUNTS):
        rows = slice(start, start + c)
        assert torch.allclose(x.grad[rows], dy[rows] @ w[e].detach(), rtol=1e-12, atol=1e-12)
        assert torch.allclose(w.grad[e], dy[rows].t() @ x[rows].detach(), rtol=1e-12, atol=1e-12)
        if c == 0:
            assert (w.grad[e] == 0).all()
        start += c


def test_grouped_swiglu_is_the_per_expert_loop():
    g = torch.Generator().manual_seed(4)
    counts = [3, 0, 5]
    x = torch.randn(8, 6, generator=g, dtype=torch.float64)
    gate, up = (torch.randn(3, 10, 6, generator=g, dtype=torch.float64) for _ in range(2))
    down = torch.randn(3, 6, 10, generator=g, dtype=torch.float64)
    got = tr.grouped_swiglu(x, gate, up, down, counts)
    silu = lambda v: v / (1 + torch.exp(-v))  # noqa: E731
    ref = torch.cat([(silu(x[:3] @ gate[0].t()) * (x[:3] @ up[0].t())) @ down[0].t(),
                     (silu(x[3:] @ gate[2].t()) * (x[3:] @ up[2].t())) @ down[2].t()])
    assert torch.allclose(got, ref, rtol=1e-12, atol=1e-12)
