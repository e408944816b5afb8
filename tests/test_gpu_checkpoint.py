"""Quantised checkpoints on the GPU: save, read without pickle, load into the
packed layout, and the layer gives the same output (tests/test_deploy_and_
distill.py:186-205 at the MoE block); static dense dispatch
(tests/test_model_features.py:49-56)."""

import numpy as np
import pytest
import torch

import oracle
import quantaweave_amd as qa
from test_checkpoint import reference_payload

pytestmark = pytest.mark.gpu


def normwise(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)


@pytest.mark.parametrize("bits,group,suffix", [(8, None, ".pt"), (4, 32, ".pt"), (4, 32, ".safetensors"),
                                               (8, None, ".safetensors")])
def test_quantized_layer_round_trips_bit_for_bit(tmp_path, bits, group, suffix):
    print(f"case checkpoint bits={bits} {suffix}", flush=True)
    torch.manual_seed(bits)
    cfg = qa.QuantaWeaveConfig(vocab_size=8, hidden_size=128, layers=1, ffn_size=96, num_experts=8, top_k=2,
                               attention_heads=1, max_sequence_length=64, capacity_factor=1.25)
    moe = qa.TopKMoE(cfg).cuda().to(torch.bfloat16)
    stats = qa.quantize_model(moe, bits, group)
    x = torch.randn(2, 40, 128, device="cuda").bfloat16()
    with torch.no_grad():
        before = moe(x)[0]
    qa.save_quantized(moe, tmp_path / f"m{suffix}", stats)
    layers = qa.load_quantized_moe(tmp_path / f"m{suffix}")
    assert list(layers) == [""]
    loaded = layers[""]
    assert loaded.experts[0].gate.qweight.dtype == (torch.int8 if bits == 8 else torch.uint8)
    assert loaded._qw_pack.fmt == (qa.moe._lib.QW_I8 if bits == 8 else qa.moe._lib.QW_U4)   # packed at load
    with torch.no_grad():
        after = loaded(x)[0]
    assert torch.equal(before, after)


def test_reference_format_checkpoint_loads_every_moe_layer(tmp_path):
    print("case checkpoint reference payload", flush=True)
    payload = reference_payload(4, 8, layers=2, E=4, D=16, F_=32)
    torch.save(payload, tmp_path / "model.int4.pt")
    layers = qa.load_quantized_moe(tmp_path / "model.int4.pt")
    assert list(layers) == ["blocks.0.moe", "blocks.1.moe"]
    x = torch.randn(24, 16, device="cuda")
    for name, moe in layers.items():
        p = name + "."
        sd = payload["state_dict"]
        w = dict(format="u4", d_model=16, d_ff=32, group_in=8, group_ff=8)
        for proj in ("gate", "up", "down"):
            w[proj] = np.stack([sd[f"{p}experts.{e}.{proj}.qweight"].numpy() for e in range(4)])
            w[proj + "_scales"] = np.stack([sd[f"{p}experts.{e}.{proj}.scales"].numpy() for e in range(4)])
        with torch.no_grad():
            out = moe(x[None])[0][0]
        ref = oracle.moe_forward(x.cpu().numpy(), sd[p + "router.weight"].numpy(), w, top_k=2, cap=48, dtype="f32")
        assert normwise(out.cpu().numpy(), ref["out"]) <= 1e-4


def small_moe(cf):
    cfg = qa.QuantaWeaveConfig(vocab_size=32, hidden_size=16, layers=2, ffn_size=32, num_experts=6, top_k=2,
                               attention_heads=2, max_sequence_length=16, capacity_factor=cf, min_expert_capacity=1)
    torch.manual_seed(1)
    return qa.TopKMoE(cfg).cuda()


def test_static_dispatch_matches_dynamic_when_capacity_is_off():
    # tests/test_model_features.py:49-56 (atol 1e-6 there; the same kernels here, so exactly equal)
    moe = small_moe(0)
    hidden = torch.randn(2, 8, 16, device="cuda")
    with torch.no_grad():
        dynamic = moe(hidden)[0]
        moe.static_dispatch = True
        static = moe(hidden)[0]
    assert torch.equal(dynamic, static)


def test_static_dispatch_ignores_capacity():
    """The dense evaluation (src/quantweave_moe_model.py:235-245) has no capacity:
    every route is evaluated, nothing overflows."""
    moe = small_moe(0.5)
    moe.static_dispatch = True
    hidden = torch.randn(3, 8, 16, device="cuda")
    with torch.no_grad():
        out, _, dropped, overflow, _ = moe(hidden)
    assert overflow.item() == 0 and dropped.item() == 0
    w = dict(format="f32", d_model=16, d_ff=32,
             gate=np.stack([e.gate.weight.detach().cpu().numpy() for e in moe.experts]),
             up=np.stack([e.up.weight.detach().cpu().numpy() for e in moe.experts]),
             down=np.stack([e.down.weight.detach().cpu().numpy() for e in moe.experts]))
    ref = oracle.moe_forward(hidden.reshape(-1, 16).cpu().numpy(), moe.router.weight.detach().cpu().numpy(), w,
                             top_k=2, cap=48, dtype="f32")
    assert normwise(out.reshape(-1, 16).cpu().numpy(), ref["out"]) <= 1e-4
