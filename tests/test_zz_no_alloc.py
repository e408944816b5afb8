"""The allocation-free decode step (qw_moe_decode_step_noalloc) against the
workspace decode step (qw_moe_decode_step), through the C ABI.

The allocation-free entry point runs the same kernels on a library-owned
static scratch array; its outputs (fp32 step output, probabilities, top-k
indices and weights) must equal the workspace call's bit for bit.  Two calls
in a row, the second with fewer tokens, check that what the first left in the
shared array does not leak into the second.
"""

import pytest
import torch

from quantaweave_amd import _hip, _lib
from quantaweave_amd import workloads as W

P = _hip.ptr


def decode_args(layer, x, residual, router):
    w = layer.w
    T = x.shape[0]
    out = torch.empty(T, w.d_model, dtype=torch.float32, device="cuda")
    probs = torch.empty(T, w.experts, dtype=torch.float32, device="cuda")
    top_idx = torch.empty(T, w.top_k, dtype=torch.int32, device="cuda")
    top_w = torch.empty(T, w.top_k, dtype=torch.float32, device="cuda")
    head = [P(x), P(residual), T, w.d_model, P(router), 1.0, P(layer.bias), w.experts, w.top_k, w.d_ff, _lib.QW_BF16,
            *layer.weight_args(), P(out), P(probs), P(top_idx), P(top_w)]
    return head, (out, probs, top_idx, top_w)


def step_noalloc(layer, x, residual, router):
    head, outs = decode_args(layer, x, residual, router)
    _lib.call("qw_moe_decode_step_noalloc", *head, _hip.stream(x.device))
    return outs


def step_workspace(layer, x, residual, router):
    w = layer.w
    head, outs = decode_args(layer, x, residual, router)
    nb = _lib.load().qw_moe_decode_step_workspace_bytes(x.shape[0], w.d_model, w.experts, w.top_k, w.d_ff,
                                                        _lib.QW_BF16)
    ws = _hip.workspace(nb, x.device)
    _lib.call("qw_moe_decode_step", *head, P(ws), nb, _hip.stream(x.device))
    return outs


@pytest.mark.gpu
@pytest.mark.parametrize("name,tokens", [("int4-decode-T16-d4096-E64-f1408-k2", (16, 3)),
                                         ("int8-decode-T64-d2048-E64-f1024-k2", (64, 1)),
                                         ("bf16-prefill-T8192-d2048-E64-f1024-k2", (40, 17))])
def test_noalloc_decode_step_equals_the_workspace_step(name, tokens):
    print(f"case noalloc decode {name} tokens={tokens}", flush=True)
    layer = W.build_layer(W.WORKLOADS[name])
    router = layer.router.float().contiguous()
    D = layer.w.d_model
    inputs = []
    for T in tokens:
        g = torch.Generator(device="cuda").manual_seed(1000 + T)
        inputs.append((torch.randn(T, D, generator=g, device="cuda"), torch.randn(T, D, generator=g, device="cuda")))
    # the allocation-free calls back to back (the second smaller), then the workspace calls
    got = [step_noalloc(layer, x, r, router) for x, r in inputs]
    want = [step_workspace(layer, x, r, router) for x, r in inputs]
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        for u, v in zip(a, b):
            assert torch.equal(u, v)
    assert got[0][0].shape[0] == tokens[0] and got[1][0].shape[0] == tokens[1]


def test_noalloc_refuses_a_step_beyond_its_scratch():
    """Sizes are checked before any device work: a step that needs more than
    the static array is refused with a clear error (no GPU needed)."""
    lib = _lib.load()
    cap = lib.qw_moe_decode_step_noalloc_scratch_bytes()
    assert cap == 32 << 20
    need = lib.qw_moe_decode_step_workspace_bytes(4096, 4096, 64, 2, 1408, _lib.QW_BF16)
    assert need > cap
    with pytest.raises(ValueError, match="scratch"):
        _lib.call("qw_moe_decode_step_noalloc", None, None, 4096, 4096, None, 1.0, None, 64, 2, 1408, _lib.QW_BF16,
                  _lib.QW_U4, 32, 32, None, None, None, None, None, None, None, None, None, None, None)
