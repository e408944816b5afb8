"""Routing and capacity plan on the GPU against the oracle — bit-exact.

Given identical fp32 logits, probabilities, top-k indices, renormalised
weights, capacity slots, dropped lists and overflow must be identical bits.
"""

import numpy as np
import pytest
import torch

import oracle
from tests import hipcall as H

pytestmark = pytest.mark.gpu


def _logits(T, E, seed, scale=2.0, hot=0.0):
    rng = np.random.RandomState(seed)
    L = (rng.randn(T, E) * scale).astype(np.float32)
    if hot:
        L[:, 0] += hot
    return L


@pytest.mark.parametrize("T,E,k", [(512, 8, 2), (8192, 64, 2), (16, 64, 2), (300, 100, 3), (257, 184, 1),
                                   (64, 1024, 8), (1, 64, 64), (33, 1, 1), (130, 65, 2)])
def test_route_from_logits_is_bit_exact(T, E, k):
    print(f"case T={T} E={E} k={k}", flush=True)
    L = _logits(T, E, T + E + k)
    p_o, i_o, w_o = oracle.route_from_logits(L, k)
    p_g, i_g, w_g = (t.cpu().numpy() for t in H.route_from_logits(H.dev(L), k))
    assert np.array_equal(p_g.view(np.int32), p_o.view(np.int32))
    assert np.array_equal(i_g, i_o)
    assert np.array_equal(w_g.view(np.int32), w_o.view(np.int32))


def test_route_with_bias_and_extreme_logits_is_bit_exact():
    L = _logits(400, 64, 5, scale=30.0)                       # probabilities down to subnormals and zero
    L[3, :] = 0.0                                             # an all-tie row
    L[4, 10:20] = 5.0                                         # ties at the top
    bias = np.linspace(-2, 2, 64).astype(np.float32)
    for b in (None, bias):
        p_o, i_o, w_o = oracle.route_from_logits(L, 4, b)
        p_g, i_g, w_g = (t.cpu().numpy() for t in H.route_from_logits(H.dev(L), 4, None if b is None else H.dev(b)))
        assert np.array_equal(p_g.view(np.int32), p_o.view(np.int32))
        assert np.array_equal(i_g, i_o) and np.array_equal(w_g.view(np.int32), w_o.view(np.int32))
    assert (p_o < 2 ** -126).any() and (p_o == 0).any()


def test_expert_bias_steers_selection_only():
    # tests/test_parallelism.py:345-357
    L = _logits(200, 4, 9)
    _, i0, w0 = H.route_from_logits(H.dev(L), 2)
    _, iz, wz = H.route_from_logits(H.dev(L), 2, H.dev(np.zeros(4, np.float32)))
    assert torch.equal(i0, iz) and torch.equal(w0, wz)
    _, ib, _ = H.route_from_logits(H.dev(L), 2, H.dev(np.float32([-100, 0, 0, 0])))
    assert (ib == 0).sum() == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T,D,E", [(512, 256, 8), (100, 2048, 64), (16, 4096, 64), (7, 33, 5),
                                   (8192, 2048, 64), (301, 192, 40), (65, 64, 1),
                                   # 16-bit router kernel: 2, 3, 5 and 8 k-chunks per wave
                                   (100, 1024, 64), (100, 1536, 48), (40, 2560, 64), (64, 4096, 64)])
def test_router_logits_match_oracle_and_routing_follows(dtype, T, D, E):
    print(f"case T={T} D={D} E={E} {dtype}", flush=True)
    g = torch.Generator().manual_seed(T + D)
    x = torch.randn(T, D, generator=g).to(dtype)
    w = (torch.randn(E, D, generator=g) * 0.02).to(dtype)
    k = min(2, E)
    logits, probs, idx, tw = H.route(x.cuda(), w.cuda(), k, temperature=1.5)
    ref = oracle.router_logits(x.float().numpy(), w.float().numpy(), 1.5)
    got = logits.cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())
    # the rest of the routing is bit-exact given the kernel's own logits
    p_o, i_o, w_o = oracle.route_from_logits(got, k)
    assert np.array_equal(probs.cpu().numpy().view(np.int32), p_o.view(np.int32))
    assert np.array_equal(idx.cpu().numpy(), i_o) and np.array_equal(tw.cpu().numpy(), w_o)



@pytest.mark.parametrize("T,D,E", [(300, 256, 64), (40, 512, 16)])
def test_router_reads_strided_rows(T, D, E):
    """x given as a view with a row stride larger than d_model gives the same bits as contiguous rows."""
    print(f"case T={T} D={D} E={E} strided", flush=True)
    g = torch.Generator().manual_seed(T * D)
    wide = torch.randn(T, D + 64, generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn(E, D, generator=g) * 0.02).to(torch.bfloat16).cuda()
    got = H.route(wide[:, :D], w, 2)
    ref = H.route(wide[:, :D].contiguous(), w, 2)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)

def _check_plan(idx, w, E, cap):
    ref = oracle.plan(idx, w, E, cap)
    got = H.plan(H.dev(idx), H.dev(w), E, cap)
    for key in ("counts", "kept_counts", "kept_offsets", "totals", "slot_token", "route_slot", "dropped_token",
                "dropped_expert"):
        assert np.array_equal(got[key], ref[key]), key
    assert np.array_equal(got["slot_weight"].view(np.int32), ref["slot_weight"].view(np.int32))
    return got


@pytest.mark.parametrize("T,E,k,cf,hot,seed", [
    (512, 8, 2, 1.25, 0.0, 0), (8192, 64, 2, 1.25, 0.0, 1), (64, 64, 2, 0.0, 0.0, 2), (16, 64, 2, 0.0, 0.0, 3),
    (4096, 64, 2, 1.0, 3.0, 4), (300, 16, 3, 0.5, 2.0, 5), (1000, 4, 1, 0.3, 0.0, 6), (9000, 1, 1, 0.5, 0.0, 7),
    (3000, 2, 2, 0.1, 0.0, 8), (5, 64, 2, 1.0, 0.0, 9), (8191, 64, 2, 1.25, 0.0, 10), (4097, 64, 2, 1.0, 3.0, 11),
    # experts past the 8192 keys the LDS sorts: the sorting network in the workspace
    (12000, 1, 1, 0.5, 0.0, 12), (20000, 8, 2, 0.3, 8.0, 13), (40000, 4, 2, 1.0, 8.0, 14),
    # more than 64 experts: the histogram from LDS atomics instead of bit-plane ballots
    (4096, 65, 2, 1.0, 3.0, 15), (3000, 100, 4, 1.25, 0.0, 16), (8192, 256, 8, 1.0, 3.0, 17),
    (2048, 1024, 2, 2.0, 0.0, 18),
])
def test_plan_is_bit_exact(T, E, k, cf, hot, seed):
    print(f"case T={T} E={E} k={k} cf={cf}", flush=True)
    _, idx, w = oracle.route_from_logits(_logits(T, E, seed, hot=hot), k)
    cap = oracle.capacity(T, k, E, cf)
    got = _check_plan(idx, w, E, cap)
    if cf and hot:
        assert got["totals"][1] > 0
    if T >= 12000:
        assert got["counts"].max() > 8192


def test_plan_with_equal_weights_and_tiny_capacity():
    T, k, E = 2000, 2, 8
    rng = np.random.RandomState(3)
    idx = np.stack([rng.choice(E, 2, replace=False) for _ in range(T)]).astype(np.int32)
    w = np.full((T, k), 0.5, np.float32)                      # every key ties on weight: route id decides
    w[::7] = np.float32([0.75, 0.25])
    for cap in (1, 4, 37, T * k):
        _check_plan(idx, w, E, cap)


def test_plan_matches_torch_double_argsort_on_device():
    """The reference's own ops (src/quantweave_moe_model.py:172-188) run by torch on the GPU."""
    T, E, k = 4096, 64, 2
    _, idx, w = oracle.route_from_logits(_logits(T, E, 11, hot=3.0), k)
    cap = oracle.capacity(T, k, E, 1.0)
    re = torch.from_numpy(idx.astype(np.int64)).cuda().reshape(-1)
    rw = torch.from_numpy(w).cuda().reshape(-1)
    by_weight = torch.argsort(rw, descending=True, stable=True)
    order = by_weight[torch.argsort(re[by_weight], stable=True)]
    counts = torch.bincount(re, minlength=E)
    offsets = torch.cumsum(counts, 0) - counts
    position = torch.arange(order.numel(), device="cuda") - offsets[re[order]]
    keep = position < cap
    got = H.plan(H.dev(idx), H.dev(w), E, cap)
    assert np.array_equal(got["slot_token"], (order[keep] // k).cpu().numpy())
    assert np.array_equal(got["dropped_token"], (order[~keep] // k).cpu().numpy())
    assert np.array_equal(got["dropped_expert"], re[order[~keep]].cpu().numpy())
    assert int(got["totals"][1]) == int((~keep).sum())


def test_empty_token_batch_is_a_no_op():
    idx = np.zeros((0, 2), np.int32)
    w = np.zeros((0, 2), np.float32)
    got = H.plan(H.dev(idx) if idx.size else torch.empty(0, 2, dtype=torch.int32, device="cuda"),
                 torch.empty(0, 2, dtype=torch.float32, device="cuda"), 8, 4)
    assert got["totals"].tolist() == [0, 0] and got["counts"].tolist() == [0] * 8
