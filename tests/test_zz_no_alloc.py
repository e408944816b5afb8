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


CAPTURE_SCRIPT = r"""
import sys
import torch
from quantaweave_amd import _hip, _lib
from quantaweave_amd import workloads as W
from tests.test_zz_no_alloc import decode_args, step_workspace

P = _hip.ptr
layer = W.build_layer(W.WORKLOADS["int4-decode-T16-d4096-E64-f1408-k2"])
router = layer.router.float().contiguous()
D = layer.w.d_model
g = torch.Generator(device="cuda").manual_seed(5)
x = torch.randn(3, D, generator=g, device="cuda")
r = torch.randn(3, D, generator=g, device="cuda")
head, outs = decode_args(layer, x, r, router)
stream = torch.cuda.Stream()
torch.cuda.synchronize()
if sys.argv[1] == "refused":
    # no set-up on this device: a call under capture must be refused, not allocate
    graph = torch.cuda.CUDAGraph()
    err = None
    with torch.cuda.graph(graph, stream=stream):
        try:
            _lib.call("qw_moe_decode_step_noalloc", *head, _hip.stream(x.device))
        except ValueError as e:
            err = str(e)
    assert err is not None and "qw_init" in err, err
    print("refused ok", flush=True)
    sys.exit(0)
_lib.call("qw_init")                               # set-up, outside capture
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=stream):       # the process's first allocation-free call
    _lib.call("qw_moe_decode_step_noalloc", *head, _hip.stream(x.device))
want = step_workspace(layer, x, r, router)
for rep in range(3):
    for t in outs:
        t.zero_()
    x.add_(0.25 * rep)                              # eager work between the replays
    want = step_workspace(layer, x, r, router)
    graph.replay()
    torch.cuda.synchronize()
    for u, v in zip(outs, want):
        assert torch.equal(u, v), rep
print("capture ok", flush=True)
"""


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["captured", "refused"])
def test_noalloc_first_call_under_graph_capture(mode):
    """A fresh process: with qw_init() made outside capture, the first
    allocation-free call is recorded in a HIP graph, and every replay (eager
    work in between) equals the workspace step bit for bit; without it, the
    call under capture is refused with an error naming qw_init."""
    import subprocess
    import sys
    from pathlib import Path

    print(f"case noalloc capture {mode}", flush=True)
    root = Path(__file__).resolve().parent.parent
    proc = subprocess.run([sys.executable, "-c", CAPTURE_SCRIPT, mode], cwd=root, capture_output=True, text=True,
                          timeout=240)
    print(proc.stdout[-2000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0
    assert ("capture ok" if mode == "captured" else "refused ok") in proc.stdout
