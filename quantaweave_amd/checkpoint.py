"""Quantised checkpoints: the reference's on-disk format read without pickle,
and its MoE layers loaded straight into the packed expert layout.

The reference writes a quantised model with ``torch.save`` of
``{"config", "bits", "group_size", "quantize_lm_head", "state_dict"}``
(``save_quantized``, src/quantization.py:105-109) and reads it back through
``torch.load(..., weights_only=False)`` (``load_quantized``, :112-117 with
src/checkpoint_io.py:23-25), which runs the file's pickle program.  Here:

* ``read_quantized`` opens the same file with ``torch.load(weights_only=True)``
  (tensors, dicts, lists, numbers and strings only: a file that holds anything
  else is refused, nothing in it is executed), or a ``.safetensors`` file
  whose header metadata carries the same fields as JSON;
* ``save_quantized`` writes either form (``.safetensors`` by suffix, else the
  reference's own ``torch.save`` payload, which the reference can load);
* ``load_quantized_moe`` builds one HIP ``TopKMoE`` per MoE layer of the
  checkpoint (a full model's ``blocks.N.moe`` or a bare layer), with int8 /
  int4 ``QuantizedLinear`` experts holding the stored bytes unchanged, and
  stacks them into the packed ``[E, out, in/2]`` device layout the expert
  kernels read.  Attention and the rest of the transformer are not part of
  this library, so the full model itself is not rebuilt.
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Optional, Union

import torch
from torch import nn

from .moe import QuantaWeaveConfig, TopKMoE, packed_experts
from .quantization import QuantizedLinear

_FIELDS = ("bits", "group_size", "quantize_lm_head")


def _config_dict(config) -> dict:
    return {k: v for k, v in dict(config.__dict__).items() if not k.startswith("_")}


def save_quantized(model: nn.Module, path: Union[str, Path], stats: dict, quantize_lm_head: bool = False) -> None:
    """src/quantization.py:105-109.  `model` needs ``.config`` (a
    QuantaWeaveConfig or the reference's) and ``state_dict()``.  A path ending in
    ``.safetensors`` gets the pickle-free form; any other path the reference's
    ``torch.save`` payload."""
    path = Path(path)
    config = _config_dict(model.config)
    state = model.state_dict()
    if path.suffix == ".safetensors":
        from safetensors.torch import save_file

        meta = {"config": json.dumps(config), "bits": json.dumps(stats["bits"]),
                "group_size": json.dumps(stats["group_size"]), "quantize_lm_head": json.dumps(bool(quantize_lm_head))}
        save_file({k: v.detach().cpu().contiguous() for k, v in state.items()}, str(path), metadata=meta)
        return
    torch.save({"config": config, "bits": stats["bits"], "group_size": stats["group_size"],
                "quantize_lm_head": quantize_lm_head, "state_dict": state}, path)


def read_quantized(path: Union[str, Path], map_location: Union[str, torch.device] = "cpu") -> dict:
    """The payload of a quantised checkpoint, read without executing anything
    from the file: {"config": dict, "bits", "group_size", "quantize_lm_head",
    "state_dict": {name: tensor}}."""
    path = Path(path)
    if path.suffix == ".safetensors":
        from safetensors import safe_open

        with safe_open(str(path), framework="pt", device="cpu") as f:
            meta = f.metadata() or {}
            state = {k: f.get_tensor(k) for k in f.keys()}
        missing = [k for k in ("config",) + _FIELDS if k not in meta]
        if missing:
            raise ValueError(f"{path} is not a quantised checkpoint (metadata lacks {missing})")
        payload = {k: json.loads(meta[k]) for k in ("config",) + _FIELDS}
        payload["state_dict"] = {k: v.to(map_location) for k, v in state.items()}
        return payload
    payload = torch.load(path, map_location=map_location, weights_only=True)
    if not isinstance(payload, dict) or "state_dict" not in payload or "config" not in payload:
        raise ValueError(f"{path} is not a quantised checkpoint")
    return payload


def _moe_prefixes(state: dict) -> list[str]:
    """Module prefixes ("blocks.0.moe." or "") of the MoE layers in a state dict."""
    suffix = "router.weight"
    return sorted({k[: -len(suffix)] for k in state if k.endswith(suffix)},
                  key=lambda p: [(0, int(t), "") if t.isdigit() else (1, 0, t) for t in p.split(".")])


def load_quantized_moe(path: Union[str, Path], device: Optional[Union[str, torch.device]] = None
                       ) -> dict[str, TopKMoE]:
    """The MoE layers of a quantised checkpoint (src/quantization.py:112-117 for
    its MoE part), keyed by module path ("blocks.0.moe"; "" for a bare layer),
    on `device` (default: the current ROCm device) in eval mode."""
    device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    payload = read_quantized(path)
    fields = {f for f in QuantaWeaveConfig.__dataclass_fields__}
    config = QuantaWeaveConfig(**{k: v for k, v in payload["config"].items() if k in fields})
    state = payload["state_dict"]
    bits, group = int(payload["bits"]), payload["group_size"]
    layers = {}
    for prefix in _moe_prefixes(state):
        moe = TopKMoE(config)
        sub = {k[len(prefix):]: v for k, v in state.items() if k.startswith(prefix)}
        for expert in moe.experts:
            for name in ("gate", "up", "down"):
                lin = getattr(expert, name)
                setattr(expert, name, QuantizedLinear(lin.in_features, lin.out_features, bits, group))
        wanted = moe.state_dict()
        missing = [k for k in wanted if k not in sub]
        if missing:
            raise ValueError(f"checkpoint lacks {prefix}{missing[0]} (and {len(missing) - 1} more)")
        for k, v in wanted.items():  # packed bytes must match exactly; float tensors may differ in dtype
            bad_dtype = sub[k].dtype != v.dtype and not (sub[k].is_floating_point() and v.is_floating_point())
            if tuple(sub[k].shape) != tuple(v.shape) or bad_dtype:
                raise ValueError(f"{prefix}{k}: stored {tuple(sub[k].shape)} {sub[k].dtype}, "
                                 f"expected {tuple(v.shape)} {v.dtype}")
        router_dtype = sub["router.weight"].dtype
        if router_dtype != moe.router.weight.dtype:
            moe.router.to(router_dtype)
        moe.load_state_dict({k: sub[k] for k in wanted})
        moe = moe.to(device).eval()
        if device.type == "cuda":
            packed_experts(moe, moe.experts)  # stacked once, in the layout the expert kernels read
        layers[prefix[:-1] if prefix.endswith(".") else prefix] = moe
    if not layers:
        raise ValueError(f"{path} holds no MoE layer (no '*router.weight')")
    return layers
