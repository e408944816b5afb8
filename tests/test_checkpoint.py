"""The quantised on-disk format (src/quantization.py:105-117) on the CPU:
the reference's torch.save payload and the safetensors form both read back
exactly, without executing anything stored in the file."""

import pickle

import numpy as np
import pytest
import torch

import oracle
import quantaweave_amd as qa
from quantaweave_amd import checkpoint


class Smuggled:
    """An object a pickle program would construct (and could run code for)."""

    def __reduce__(self):
        return (print, ("this must never run",))


def reference_payload(bits, group, layers=2, E=4, D=16, F_=32):
    """The dict the reference's save_quantized writes for a small model: config,
    bits, group size and a state dict with blocks.N.moe.* quantised experts
    (packed with the oracle's quantiser) plus a non-MoE tensor."""
    cfg = qa.QuantaWeaveConfig(vocab_size=32, hidden_size=D, layers=layers, ffn_size=F_, num_experts=E, top_k=2,
                               attention_heads=2, max_sequence_length=16, capacity_factor=0)
    rng = np.random.default_rng(bits)
    state = {"embed.weight": torch.randn(32, D)}
    for b in range(layers):
        p = f"blocks.{b}.moe."
        state[p + "router.weight"] = torch.from_numpy(rng.standard_normal((E, D)).astype(np.float32))
        for e in range(E):
            for name, (o, i) in (("gate", (F_, D)), ("up", (F_, D)), ("down", (D, F_))):
                q, s, _ = oracle.quantize(rng.standard_normal((o, i)).astype(np.float32), bits, group)
                state[f"{p}experts.{e}.{name}.qweight"] = torch.from_numpy(q)
                state[f"{p}experts.{e}.{name}.scales"] = torch.from_numpy(s)
    return {"config": dict(cfg.__dict__), "bits": bits, "group_size": group, "quantize_lm_head": False,
            "state_dict": state}


@pytest.mark.parametrize("bits,group", [(8, None), (4, 8)])
def test_reference_payload_reads_back_exactly(tmp_path, bits, group):
    payload = reference_payload(bits, group)
    torch.save(payload, tmp_path / "m.pt")
    got = checkpoint.read_quantized(tmp_path / "m.pt")
    assert got["bits"] == bits and got["group_size"] == group and got["config"] == payload["config"]
    assert set(got["state_dict"]) == set(payload["state_dict"])
    for k, v in payload["state_dict"].items():
        assert got["state_dict"][k].dtype == v.dtype and torch.equal(got["state_dict"][k], v)
    assert checkpoint._moe_prefixes(got["state_dict"]) == ["blocks.0.moe.", "blocks.1.moe."]


def test_safetensors_form_round_trips(tmp_path):
    payload = reference_payload(4, 8)

    class Holder(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.config = qa.QuantaWeaveConfig(**payload["config"])
            for k, v in payload["state_dict"].items():
                self.register_buffer(k.replace(".", "__"), v)

        def state_dict(self, *a, **kw):
            return payload["state_dict"]

    qa.save_quantized(Holder(), tmp_path / "m.safetensors", {"bits": 4, "group_size": 8})
    got = qa.read_quantized(tmp_path / "m.safetensors")
    assert got["bits"] == 4 and got["group_size"] == 8 and got["quantize_lm_head"] is False
    assert got["config"] == payload["config"]
    for k, v in payload["state_dict"].items():
        assert torch.equal(got["state_dict"][k], v)


def test_a_file_holding_code_is_refused_and_nothing_runs(tmp_path, capsys):
    torch.save({"config": {}, "state_dict": {}, "bits": 8, "group_size": None, "quantize_lm_head": False,
                "extra": Smuggled()}, tmp_path / "evil.pt")
    with pytest.raises(pickle.UnpicklingError):
        checkpoint.read_quantized(tmp_path / "evil.pt")
    assert "must never run" not in capsys.readouterr().out


def test_not_a_checkpoint_is_reported(tmp_path):
    torch.save({"weights": torch.zeros(2)}, tmp_path / "x.pt")
    with pytest.raises(ValueError, match="not a quantised checkpoint"):
        checkpoint.read_quantized(tmp_path / "x.pt")
