"""Routed MoE layer — drop-in for QuantaWeave's ``TopKMoE`` on MI355X.

``TopKMoE`` keeps the reference module's constructor, parameters
(``router``, ``experts[i].{gate,up,down}``), runtime switches and forward
signature (src/quantweave_moe_model.py:63-272).  Its forward is one call into
the C ABI (``qw_moe_forward``): router, softmax/top-k, capacity plan, grouped
SwiGLU experts and the weighted combine all run as HIP kernels on the current
stream, with no host synchronisation.  With autograd on and float experts,
the same kernels run inside ``_MoELayer`` (one C call per stage, outputs
identical to the inference call, the experts keeping their activations),
whose backward runs the grouped backward kernels.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from itertools import chain
from operator import attrgetter, itemgetter, methodcaller
from typing import Optional

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import _hip, _lib
from .quantization import QuantizedLinear


@dataclass
class QuantaWeaveConfig:
    """Same fields, defaults and validation as src/quantweave_moe_model.py:15-48."""

    vocab_size: int = 7168
    hidden_size: int = 64
    layers: int = 2
    ffn_size: int = 128
    num_experts: int = 184
    top_k: int = 1
    attention_heads: int = 4
    max_sequence_length: int = 256
    router_aux_loss_coef: float = 0.01
    capacity_factor: float = 1.25
    min_expert_capacity: int = 4
    drop_overflow_tokens: bool = True
    overflow_policy: str = "drop"
    router_temperature: float = 1.0

    def __post_init__(self) -> None:
        if self.vocab_size < 2 or self.hidden_size < 1 or self.layers < 1:
            raise ValueError("vocab_size, hidden_size, and layers must be positive")
        if self.ffn_size < 1 or self.attention_heads < 1:
            raise ValueError("ffn_size and attention_heads must be positive")
        if self.hidden_size % self.attention_heads:
            raise ValueError("hidden_size must be divisible by attention_heads")
        if self.num_experts < 1 or not 1 <= self.top_k <= self.num_experts:
            raise ValueError("top_k must be between 1 and num_experts")
        if self.max_sequence_length < 2:
            raise ValueError("max_sequence_length must be at least 2")
        if self.capacity_factor < 0 or self.min_expert_capacity < 1:
            raise ValueError("capacity_factor must be >= 0 and min_expert_capacity must be positive")
        if self.overflow_policy not in {"drop", "residual"}:
            raise ValueError("overflow_policy must be 'drop' or 'residual'")
        if self.router_temperature <= 0:
            raise ValueError("router_temperature must be positive")


class SparseSwiGLU(nn.Module):
    """down(silu(gate(x)) * up(x)) with bias-free projections (src/quantweave_moe_model.py:51-60).

    Holds the parameters of one expert; TopKMoE evaluates all experts together
    in the grouped HIP kernels.  Calling an expert on its own runs the grouped
    kernel with one expert."""

    def __init__(self, config, ffn_size: Optional[int] = None) -> None:
        super().__init__()
        ffn_size = ffn_size or config.ffn_size
        self.gate = nn.Linear(config.hidden_size, ffn_size, bias=False)
        self.up = nn.Linear(config.hidden_size, ffn_size, bias=False)
        self.down = nn.Linear(ffn_size, config.hidden_size, bias=False)

    def forward(self, hidden: Tensor) -> Tensor:
        from .moe_kernels import grouped_swiglu

        lead = hidden.shape[:-1]
        flat = hidden.reshape(-1, hidden.size(-1))
        return grouped_swiglu(flat, nn.ModuleList([self]), [flat.size(0)]).reshape(*lead, -1)


def _expert_format(experts: nn.ModuleList) -> tuple[int, int, int]:
    """(weight format, gate/up group, down group) shared by every projection."""
    first = experts[0].gate
    if isinstance(first, QuantizedLinear):
        fmt = first.w_format
        g_in, g_ff = first.group_size, experts[0].down.group_size
        for e in experts:
            for name, g in (("gate", g_in), ("up", g_in), ("down", g_ff)):
                p = getattr(e, name)
                if not isinstance(p, QuantizedLinear) or p.w_format != fmt or p.group_size != g:
                    raise ValueError("all experts must share one quantisation format and group size")
        return fmt, g_in, g_ff
    dt = first.weight.dtype
    for e in experts:
        for name in ("gate", "up", "down"):
            p = getattr(e, name)
            if not isinstance(p, nn.Linear) or p.bias is not None or p.weight.dtype != dt:
                raise ValueError("experts must be bias-free nn.Linear (one dtype) or QuantizedLinear projections")
    if dt not in _hip.FLOAT_DTYPES:
        raise ValueError(f"expert weight dtype {dt} is not supported (float32, bfloat16 or float16)")
    return _hip.act_code(first.weight, "experts"), 0, 0


def tile_bf16(stack: Tensor) -> Tensor:
    """bf16 (or fp16) weights [E, out, in] (nn.Linear layout) rearranged into
    the 1 KiB tiles of QW_BF16T (QW_F16T) (qw_pack_bf16_tiles); same shape and size."""
    stack = stack.contiguous()
    _hip.require_device(stack, "tile_bf16")
    if stack.dtype not in _hip.HALF or stack.dim() != 3:
        raise ValueError("tile_bf16 takes a bf16 or fp16 [experts, out, in] tensor")
    out = torch.empty_like(stack)
    E, rows, cols = stack.shape
    _lib.call("qw_pack_bf16_tiles", _hip.ptr(stack), E, rows, cols, _hip.ptr(out), _hip.stream(stack.device))
    return out


def can_tile(stack: Tensor) -> bool:
    return stack.dtype in _hip.HALF and stack.size(1) % 64 == 0 and stack.size(2) % 64 == 0


# Every registration of a module, parameter or buffer anywhere in the process
# (nn.Module.__setattr__, add_module, register_parameter / register_buffer)
# bumps this generation.  An expert pack that recorded the current generation
# knows that no expert module, weight or buffer object was swapped since.
_GENERATION = [0]


def _registered(*_args) -> None:
    _GENERATION[0] += 1


_REGISTRATION_HOOKS = (
    torch.nn.modules.module.register_module_module_registration_hook(_registered),
    torch.nn.modules.module.register_module_parameter_registration_hook(_registered),
    torch.nn.modules.module.register_module_buffer_registration_hook(_registered),
)

_SUBMODULES = attrgetter("_modules")
_GATE_UP_DOWN = itemgetter("gate", "up", "down")
_PARAMETERS = attrgetter("_parameters")
_BUFFERS = attrgetter("_buffers")
_WEIGHT = itemgetter("weight")
_QBUFFERS = itemgetter("qweight", "scales")
_VERSION = attrgetter("_version")
_DATA_PTR = methodcaller("data_ptr")
_REQUIRES_GRAD = attrgetter("requires_grad")


class ExpertPack:
    """Experts' weights stacked once into [E, out, in] device buffers.

    Replaces the per-call ``torch.stack`` of src/moe_kernels.py:191-193; the pack
    is rebuilt only when a projection module, parameter or buffer changes.
    bf16 and fp16 weights whose shapes allow it are kept in the QW_BF16T /
    QW_F16T tiles the prefill kernels stream contiguously.

    Quantised experts' ``qweight`` / ``scales`` buffers are re-registered as
    views of the pack's stacks (``rehome``): the module and the kernels then
    read one copy of the bytes.

    Currency, per call: ``fast_current`` when the pack is armed, else
    ``current``.  ``current`` compares every module, tensor, version counter
    and storage pointer (O(experts)).  ``arm`` makes an O(1) token when the
    experts' tensors share a few version counters (float weights created by
    TopKMoE as views of one buffer, quantised buffers re-homed into the
    stacks): the registration generation, those counters' versions and the
    first and last tensor's identity and storage.  What the token cannot see:
    replacing one expert tensor's storage without registering anything (an
    ``_apply`` on a single expert, ``.data =`` on one weight); call
    ``TopKMoE.refresh_experts()`` after such a change."""

    def __init__(self, experts: nn.ModuleList, rehome: bool = True) -> None:
        self.fmt, self.group_in, self.group_ff = _expert_format(experts)
        self._exps = tuple(experts._modules.values())
        self._quant = isinstance(self._exps[0]._modules["gate"], QuantizedLinear)
        self._token = None
        if self.fmt in (_lib.QW_F32, _lib.QW_BF16, _lib.QW_F16):
            self.gate = torch.stack([e.gate.weight.detach() for e in experts]).contiguous()
            self.up = torch.stack([e.up.weight.detach() for e in experts]).contiguous()
            self.down = torch.stack([e.down.weight.detach() for e in experts]).contiguous()
            self.gate_s = self.up_s = self.down_s = None
            self.maybe_tile()
        else:
            self.gate = torch.stack([e.gate.qweight for e in experts]).contiguous()
            self.up = torch.stack([e.up.qweight for e in experts]).contiguous()
            self.down = torch.stack([e.down.qweight for e in experts]).contiguous()
            self.gate_s = torch.stack([e.gate.scales.float() for e in experts]).contiguous()
            self.up_s = torch.stack([e.up.scales.float() for e in experts]).contiguous()
            self.down_s = torch.stack([e.down.scales.float() for e in experts]).contiguous()
            if rehome and self.gate.device.type == "cuda":
                for i, e in enumerate(self._exps):
                    for name, q, sc in (("gate", self.gate, self.gate_s), ("up", self.up, self.up_s),
                                        ("down", self.down, self.down_s)):
                        m = e._modules[name]
                        m.qweight, m.scales = q[i], sc[i]
        self._record(experts)

    def _record(self, experts: nn.ModuleList) -> None:
        """What ``current`` compares, as tuples built by C-level iteration (the
        pack holds the objects, so their ids cannot be reused meanwhile)."""
        self.mods, self.tensors = ExpertPack.sources(experts)
        self._exp_ids = tuple(map(id, self._exps))
        self._mod_ids = tuple(map(id, self.mods))
        self._tensor_ids = tuple(map(id, self.tensors))
        self.versions = tuple(map(_VERSION, self.tensors))
        self.ptrs = tuple(map(_DATA_PTR, self.tensors))

    def __getstate__(self) -> dict:
        state = dict(self.__dict__)
        state["_token"] = None  # a copy's tensors may not share counters: re-armed on first use
        return state

    def arm(self) -> None:
        """Make the O(1) token if the pack's tensors share at most 8 version
        counters.  Sharing is found by bumping each candidate counter once
        (torch.autograd.graph.increment_version: no data is touched) and
        seeing which tensors' versions move with it."""
        self._token = None
        reps, rest = [], list(self.tensors)
        while rest and len(reps) < 8:
            before = tuple(map(_VERSION, rest))
            torch.autograd.graph.increment_version(rest[0])
            after = tuple(map(_VERSION, rest))
            reps.append(rest[0])
            rest = [t for t, b, a in zip(rest, before, after) if a == b]
        self.versions = tuple(map(_VERSION, self.tensors))
        if rest:
            return
        self._reps = tuple(reps)
        first, last = self.tensors[0], self.tensors[-1]
        self._token = (_GENERATION[0], tuple(map(_VERSION, self._reps)), first.data_ptr(), last.data_ptr())

    def fast_current(self) -> bool:
        """The O(1) check of an armed pack (see the class docstring)."""
        tok = self._token
        if tok is None or tok[0] != _GENERATION[0] or tuple(map(_VERSION, self._reps)) != tok[1]:
            return False
        e0, e1 = self._exps[0]._modules, self._exps[-1]._modules
        if self._quant:
            first, last = e0["gate"]._buffers["qweight"], e1["down"]._buffers["scales"]
        else:
            first, last = e0["gate"]._parameters["weight"], e1["down"]._parameters["weight"]
        return (first is self.tensors[0] and last is self.tensors[-1] and first.data_ptr() == tok[2]
                and last.data_ptr() == tok[3])

    def maybe_tile(self) -> None:
        """bf16 / fp16 stacks on a ROCm device -> QW_BF16T / QW_F16T tiles (in place of the plain stacks)."""
        if self.fmt not in (_lib.QW_BF16, _lib.QW_F16) or self.gate.device.type != "cuda":
            return
        if all(can_tile(t) for t in (self.gate, self.up, self.down)):
            self.gate, self.up, self.down = tile_bf16(self.gate), tile_bf16(self.up), tile_bf16(self.down)
            self.fmt = _lib.QW_BF16T if self.fmt == _lib.QW_BF16 else _lib.QW_F16T

    @staticmethod
    def sources(experts: nn.ModuleList) -> tuple[list, list]:
        """The projection modules and the tensors the pack was made from."""
        mods = [m for e in experts._modules.values() for m in (e._modules["gate"], e._modules["up"], e._modules["down"])]
        tensors = []
        for m in mods:
            if isinstance(m, QuantizedLinear):
                tensors += (m._buffers["qweight"], m._buffers["scales"])
            else:
                tensors.append(m._parameters["weight"])
        return mods, tensors

    def current(self, experts: nn.ModuleList) -> bool:
        """True while the experts hold the same modules and tensors, unmodified
        (same storage, same version counter): the per-call check."""
        if tuple(map(id, experts._modules.values())) != self._exp_ids:
            return False
        mods = tuple(chain.from_iterable(map(_GATE_UP_DOWN, map(_SUBMODULES, self._exps))))
        if tuple(map(id, mods)) != self._mod_ids:
            return False
        if self._quant:
            tensors = chain.from_iterable(map(_QBUFFERS, map(_BUFFERS, mods)))
        else:
            tensors = map(_WEIGHT, map(_PARAMETERS, mods))
        if tuple(map(id, tensors)) != self._tensor_ids:
            return False
        return (tuple(map(_VERSION, self.tensors)) == self.versions
                and tuple(map(_DATA_PTR, self.tensors)) == self.ptrs)

    def args(self) -> tuple:
        """Weight arguments of the C ABI (format, groups, weight and scale
        pointers), kept while the pack holds the same tensors."""
        key = (self.fmt, id(self.gate), id(self.up), id(self.down), id(self.gate_s), id(self.up_s), id(self.down_s))
        cached = self.__dict__.get("_args")
        if cached is None or cached[0] != key:
            cached = (key, (self.fmt, self.group_in, self.group_ff, _hip.ptr(self.gate), _hip.ptr(self.gate_s),
                            _hip.ptr(self.up), _hip.ptr(self.up_s), _hip.ptr(self.down), _hip.ptr(self.down_s)))
            self._args = cached
        return cached[1]

    def plain(self, experts: nn.ModuleList, dtype: torch.dtype) -> list:
        """[gate, up, down] stacks [E, out, in] in `dtype`, untiled, for the
        backward kernels; made once per weight version."""
        cache = getattr(self, "_plain", None)
        if cache is None or cache[0] != dtype:
            stacks = [torch.stack([getattr(e, n).weight.detach() for e in experts]).to(dtype).contiguous()
                      for n in ("gate", "up", "down")]
            cache = (dtype, stacks)
            self._plain = cache
        return cache[1]

    def args_for(self, act: int) -> list:
        """Weight arguments for activations of dtype code `act`: float experts
        multiplied in another 16-bit type (fp32 experts under bf16 or fp16
        autocast, bf16 experts under fp16 autocast and the reverse) use copies
        in that type (tiled where the shapes allow), made once per weight
        version — the reference's per-call ``stack(...).to(dtype)``
        (src/moe_kernels.py:191-193)."""
        return self.for_act(act).args()

    def for_act(self, act: int) -> "ExpertPack":
        """This pack, or its copy in the 16-bit activation type `act`."""
        plain_of = {_lib.QW_BF16T: _lib.QW_BF16, _lib.QW_F16T: _lib.QW_F16}
        src = plain_of.get(self.fmt, self.fmt)
        if act not in (_lib.QW_BF16, _lib.QW_F16) or src not in (_lib.QW_F32, _lib.QW_BF16, _lib.QW_F16) or src == act:
            return self
        copies = self.__dict__.setdefault("_copies", {})
        if act not in copies:
            dt = torch.bfloat16 if act == _lib.QW_BF16 else torch.float16
            cast = ExpertPack.__new__(ExpertPack)
            cast.group_in, cast.group_ff = 0, 0
            # tiles are a permutation of the elements: a cast keeps them tiles
            cast.gate, cast.up, cast.down = (t.to(dt).contiguous() for t in (self.gate, self.up, self.down))
            cast.gate_s = cast.up_s = cast.down_s = None
            if self.fmt in plain_of:
                cast.fmt = _lib.QW_BF16T if act == _lib.QW_BF16 else _lib.QW_F16T
            else:
                cast.fmt = act
                cast.maybe_tile()
            copies[act] = cast
        return copies[act]

    def expert_args(self, e: int) -> list:
        """Weight arguments of expert e alone (views into the stacks)."""
        def one(t):
            return None if t is None else _hip.ptr(t[e])

        return [self.fmt, self.group_in, self.group_ff, one(self.gate), one(self.gate_s), one(self.up),
                one(self.up_s), one(self.down), one(self.down_s)]


def packed_experts(owner: nn.Module, experts: nn.ModuleList) -> ExpertPack:
    """The owner's expert pack, rebuilt when the experts changed: an armed
    pack is checked in O(1), otherwise every expert tensor is compared and the
    pack re-armed."""
    pack = owner.__dict__.get("_qw_pack")
    if pack is not None and pack.fast_current():
        return pack
    if pack is None or not pack.current(experts):
        pack = ExpertPack(experts)
        owner._qw_pack = pack
    pack.arm()
    return pack


class TopKMoE(nn.Module):
    """Top-k routed mixture of SwiGLU experts (src/quantweave_moe_model.py:63-272).

    Routing runs in fp32.  Routes are ordered by (expert, -weight, route id) and
    each expert keeps its first ``capacity`` routes; the others are skipped and
    reported as overflow (and as dropped under the "drop" policy).
    """

    def __init__(self, config, num_local_experts: Optional[int] = None, tensor_parallel=None) -> None:
        super().__init__()
        if config.top_k < 1 or config.top_k > config.num_experts:
            raise ValueError("top_k must be between 1 and num_experts")
        self.tp_size = getattr(tensor_parallel, "tp_size", 1)
        if self.tp_size > 1:
            raise ValueError("tensor-parallel MoE is not supported by the single-GPU HIP path")
        self.tp_group = None
        self.config = config  # kept for save_quantized of a bare layer
        self.num_experts = config.num_experts
        self.top_k = config.top_k
        self.capacity_factor = config.capacity_factor
        self.min_expert_capacity = config.min_expert_capacity
        self.drop_overflow_tokens = config.drop_overflow_tokens
        self.overflow_policy = config.overflow_policy
        self.router_temperature = config.router_temperature
        self.router = nn.Linear(config.hidden_size, config.num_experts, bias=False)
        self.num_local_experts = num_local_experts or config.num_experts
        if self.num_local_experts != self.num_experts:
            raise ValueError("expert-parallel sharding is not supported by the single-GPU HIP path")
        self.experts = nn.ModuleList(SparseSwiGLU(config, config.ffn_size) for _ in range(self.num_local_experts))
        self._share_expert_storage()
        # runtime switches (not parameters or saved state), as in the reference
        self.collect_stats = False
        self.static_dispatch = False
        self.profile_experts = False
        self.use_triton_kernels = True  # grouped kernels are the only executor here
        self.expert_bias: Optional[Tensor] = None
        self.capacity_scale: float = 1.0
        self.expert_seconds = [0.0] * self.num_local_experts
        self.last_top_indices: Optional[Tensor] = None
        self.last_stats: dict[str, Tensor] = {}
        self.last_plan: dict[str, Tensor] = {}

    @property
    def last_top_indices(self) -> Optional[Tensor]:
        """The last forward's expert choices [tokens, top_k], int64 as the
        reference stores them (src/quantweave_moe_model.py:137).  The forward
        keeps the kernel's int32 choices (a fresh tensor per call) and widens
        them on first read, so a forward whose choices nobody reads launches
        no conversion."""
        v = self.__dict__.get("_last_top_idx")
        if v is not None and v.dtype != torch.long:
            v = v.long()
            self.__dict__["_last_top_idx"] = v
        return v

    @last_top_indices.setter
    def last_top_indices(self, value: Optional[Tensor]) -> None:
        self.__dict__["_last_top_idx"] = value

    @torch.no_grad()
    def _share_expert_storage(self) -> None:
        """Re-create the experts' weights (same values, shapes and
        requires_grad) as views of one buffer.  Views of one tensor share its
        version counter, and keep sharing it through .to() / .cuda() / .half()
        (which swap each parameter's data in place), so the expert pack's
        per-call check reads one version instead of one per weight."""
        lins = [e._modules[n] for e in self.experts for n in ("gate", "up", "down")]
        ws = [lin._parameters["weight"] for lin in lins]
        base = torch.empty(sum(w.numel() for w in ws), dtype=ws[0].dtype, device=ws[0].device)
        off = 0
        for lin, w in zip(lins, ws):
            view = base[off:off + w.numel()].view_as(w)
            view.copy_(w)
            lin.weight = nn.Parameter(view, requires_grad=w.requires_grad)
            off += w.numel()

    def refresh_experts(self) -> None:
        """Drop the expert pack, so the next forward re-stacks the experts'
        weights.  Needed only after a change the pack's checks cannot see:
        ``.data =`` on one expert weight, or ``.to()`` applied to a single
        expert."""
        self.__dict__.pop("_qw_pack", None)

    def capacity(self, num_tokens: int) -> int:
        """Route slots per expert (src/quantweave_moe_model.py:100-111)."""
        if self.capacity_factor > 0 and self.drop_overflow_tokens:
            return max(
                self.min_expert_capacity,
                math.ceil(num_tokens * self.top_k / self.num_experts * self.capacity_factor * self.capacity_scale),
            )
        return num_tokens * self.top_k

    def _wants_grad(self, hidden: Tensor, pack: "ExpertPack") -> bool:
        if not torch.is_grad_enabled():
            return False
        if hidden.requires_grad or self.router.weight.requires_grad:
            return True
        if pack._quant:
            return False
        return any(map(_REQUIRES_GRAD, pack.tensors))

    def forward(self, hidden: Tensor, token_domains: Optional[Tensor] = None,
                num_domains: int = 0) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
        """Returns (output, balance_loss, dropped_routes, overflow_routes, domain_loss)."""
        _hip.require_device(hidden, "TopKMoE.forward")
        batch, sequence, width = hidden.shape
        flat = hidden.reshape(-1, width)
        act = _hip.act_code(flat, "TopKMoE.forward")
        dev = flat.device
        T, E, K = flat.size(0), self.num_experts, self.top_k
        bias = None
        if self.expert_bias is not None:
            bias = self.expert_bias.detach().to(dev, torch.float32).contiguous()
        pack = packed_experts(self, self.experts)
        # static dispatch is the capacity-free evaluation (src/quantweave_moe_model.py:235-245),
        # with its own accumulation (route weights cast to the hidden dtype, a rounding per add)
        static = bool(self.static_dispatch)
        cap = T * K if static else self.capacity(T)
        cdt = _compute_dtype(flat)
        # per-expert timing (profile_experts) runs the experts one call at a time and
        # records no autograd graph; an input that requires grad keeps the graph instead
        profiling = self.profile_experts and not (hidden.requires_grad and torch.is_grad_enabled())
        # the loop executor (use_triton_kernels False, set_moe_kernel("loop")) launches
        # the experts one at a time, as the reference's loop does (:203-209)
        loop = not self.use_triton_kernels
        if not profiling and self._wants_grad(hidden, pack):
            if pack.fmt not in (_lib.QW_F32, _lib.QW_BF16, _lib.QW_BF16T, _lib.QW_F16, _lib.QW_F16T):
                if hidden.requires_grad:
                    raise NotImplementedError("gradients through quantised experts are not supported")
            else:
                weights = [getattr(e, n).weight for e in self.experts for n in ("gate", "up", "down")]
                out, probs, balance, top_idx, top_w, counts, kept_counts, totals, dropped_token, dropped_expert = \
                    _MoELayer.apply(flat, self.router.weight, self, pack, cap, bias, cdt, loop, static, *weights)
                return self._finish(out, probs, balance, top_idx, top_w, counts, kept_counts, totals, dropped_token,
                                    dropped_expert, token_domains, num_domains, (batch, sequence, width))
        with torch.no_grad():
            flat = flat.detach().contiguous()
            if profiling:
                res = _layer_chain(flat, cdt, self.router.weight, self, pack, cap, bias, loop=True, static=static,
                                   profile=self.expert_seconds)
            elif cdt == flat.dtype and not loop and not static:
                res = _forward_call(flat, act, self.router.weight, self, pack, cap, bias)
            else:
                res = _layer_chain(flat, cdt, self.router.weight, self, pack, cap, bias, loop=loop, static=static)
        return self._finish(res["out"], res["probs"], res["balance"], res["top_idx"], res["top_w"], res["counts"],
                            res["kept_counts"], res["totals"], res["dropped_token"], res["dropped_expert"],
                            token_domains, num_domains, (batch, sequence, width))

    def _finish(self, out, probs, balance, top_idx, top_w, counts, kept_counts, totals, dropped_token, dropped_expert,
                token_domains, num_domains, shape):
        dev = out.device
        self.last_top_indices = top_idx  # widened to int64 when read
        self.last_plan = dict(counts=counts, kept_counts=kept_counts, totals=totals, top_w=top_w,
                              dropped_token=dropped_token, dropped_expert=dropped_expert)
        overflow_routes = totals[1].long()
        if self.overflow_policy == "drop":
            dropped_routes = overflow_routes
        else:
            dropped_routes = torch.zeros((), device=dev, dtype=torch.long)
        if self.collect_stats and not self.static_dispatch:  # the dynamic path only (:141-149)
            self._record_stats(probs.detach(), top_idx, kept_counts, totals, dropped_token, dropped_expert)
        domain_loss = probs.new_zeros(())
        if token_domains is not None and num_domains > 1:
            domain_loss = self._domain_loss(probs, token_domains, num_domains)
        return out.reshape(*shape), balance, dropped_routes, overflow_routes, domain_loss

    def _domain_loss(self, router_probs: Tensor, token_domains: Tensor, num_domains: int) -> Tensor:
        """Mean pairwise cosine similarity of the domains' routing profiles
        (src/quantweave_moe_model.py:247-257); an auxiliary loss off the FFN path."""
        membership = F.one_hot(token_domains.reshape(-1).long(), num_domains).to(router_probs.dtype)
        counts = membership.sum(dim=0)
        profiles = (membership.t() @ router_probs) / counts.clamp(min=1)[:, None]
        profiles = F.normalize(profiles[counts > 0], dim=-1)
        present = profiles.size(0)
        if present < 2:
            return router_probs.new_zeros(())
        similarity = profiles @ profiles.t()
        return (similarity.sum() - similarity.diagonal().sum()) / (present * (present - 1))

    @torch.no_grad()
    def _record_stats(self, router_probs, top_indices, kept_counts, totals, dropped_token, dropped_expert) -> None:
        """src/quantweave_moe_model.py:259-272 (reads the dropped count back to size the lists)."""
        entropy = -(router_probs * router_probs.clamp_min(1e-12).log()).sum(dim=-1)
        top_probability = router_probs.max(dim=-1).values
        n_drop = int(totals[1].item())
        self.last_stats = {
            "expert_load": kept_counts.long(),
            "expert_assigned": torch.bincount(top_indices.reshape(-1).long(), minlength=self.num_experts),
            "importance": router_probs.mean(dim=0),
            "entropy_mean": entropy.mean(),
            "confidence_mean": top_probability.mean(),
            "confidence_hist": torch.histc(top_probability.float(), bins=10, min=0.0, max=1.0),
            "dropped_tokens": dropped_token[:n_drop].long(),
            "dropped_experts": dropped_expert[:n_drop].long(),
        }


def _router_operand(router_w: Tensor) -> Tensor:
    w = router_w.detach()
    if w.dtype not in _hip.FLOAT_DTYPES:
        w = w.float()
    return w.contiguous()


def _forward_call(flat: Tensor, act: int, router_w: Tensor, moe: TopKMoE, pack: ExpertPack, cap: int,
                  bias: Optional[Tensor]) -> dict:
    """The whole layer forward as one qw_moe_forward call (inference)."""
    dev = flat.device
    T, width = flat.shape
    E, K = moe.num_experts, moe.top_k
    R = T * K
    Rm = max(R, 1)
    rw = _router_operand(router_w)
    # the per-call outputs in two slabs (int32 and fp32), handed out as views
    ints = torch.empty(R + 2 * E + 2 + 2 * Rm, dtype=torch.int32, device=dev)
    flts = torch.empty(T * E + R + 1 + E, dtype=torch.float32, device=dev)
    top_idx, counts, kept_counts, totals, dropped_token, dropped_expert = ints.split([R, E, E, 2, Rm, Rm])
    probs, top_w, balance, importance = flts.split([T * E, R, 1, E])
    r = dict(out=torch.empty_like(flat), probs=probs.view(T, E), top_w=top_w.view(T, K), balance=balance.view(()),
             top_idx=top_idx.view(T, K), counts=counts, kept_counts=kept_counts, totals=totals,
             dropped_token=dropped_token, dropped_expert=dropped_expert)
    if not T:
        totals.zero_()
        balance.zero_()
        return r
    key = (T, width, E, K, act)
    sizes = moe.__dict__.setdefault("_qw_sizes", {}).get(key)
    lib = _lib.load()
    if sizes is None:
        d_ff = moe.experts[0].gate.out_features
        nbytes = lib.qw_moe_forward_workspace_bytes(T, width, E, K, d_ff, act)
        fwd_bytes = (nbytes + 255) // 256 * 256
        sizes = (d_ff, nbytes, fwd_bytes, lib.qw_moe_balance_workspace_bytes(T, E))
        moe._qw_sizes[key] = sizes
    d_ff, nbytes, fwd_bytes, bal_bytes = sizes
    s = torch.cuda.current_stream(dev).cuda_stream
    ws = _stream_workspace(moe, fwd_bytes + bal_bytes, dev, s)
    wp, ip, fp = ws.data_ptr(), ints.data_ptr(), flts.data_ptr()
    p_probs, p_counts = fp, ip + 4 * (R + 0)
    _lib.check(lib.qw_moe_forward(
        flat.data_ptr(), act, T, width, rw.data_ptr(), _hip.act_code(rw, "router"), float(moe.router_temperature),
        _hip.ptr(bias), E, K, cap, d_ff, *pack.args(), r["out"].data_ptr(), p_probs, ip, fp + 4 * T * E, p_counts,
        ip + 4 * (R + E), ip + 4 * (R + 2 * E), ip + 4 * (R + 2 * E + 2), ip + 4 * (R + 2 * E + 2 + Rm), wp, nbytes,
        s), "qw_moe_forward")
    _lib.check(lib.qw_moe_balance_ws(p_probs, p_counts, T, K, E, fp + 4 * (T * E + R + 1), fp + 4 * (T * E + R), wp +
                                     fwd_bytes, bal_bytes, s), "qw_moe_balance_ws")
    return r


def _stream_workspace(moe: nn.Module, nbytes: int, dev: torch.device, stream: int) -> Tensor:
    """The module's forward workspace for `stream` (the current one), kept
    between calls (calls on one stream are ordered, so one buffer serves them
    all; a call on another stream gets its own).  Grown when a call needs more."""
    cache = moe.__dict__.setdefault("_qw_workspaces", {})
    key = (dev, stream)
    ws = cache.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = _hip.workspace(nbytes, dev)
        cache[key] = ws
    return ws


def _compute_dtype(flat: Tensor) -> torch.dtype:
    """The experts' arithmetic dtype: the autocast dtype when autocast is on,
    else the input dtype (src/moe_kernels.py:179-183): fp32, bf16 or fp16."""
    dt = flat.dtype
    if torch.is_autocast_enabled(flat.device.type):
        dt = torch.get_autocast_dtype(flat.device.type)
    if dt not in _hip.FLOAT_DTYPES:
        raise ValueError(f"TopKMoE.forward: compute dtype {dt} is not supported (float32, bfloat16 or float16)")
    return dt


def _layer_chain(flat: Tensor, cdt: torch.dtype, router_w: Tensor, moe: TopKMoE, pack: ExpertPack, cap: int,
                 bias: Optional[Tensor], save: bool = False, loop: bool = False, static: bool = False,
                 profile: Optional[list] = None) -> dict:
    """The layer forward as one C call per stage: qw_moe_route (on the input
    dtype, src/quantweave_moe_model.py:126-127), qw_moe_plan, qw_moe_experts
    on the rows cast to `cdt` (unweighted rows) and qw_moe_combine_weighted,
    which forms `(expert_output * weights[:, None]).to(output.dtype)` and adds
    it in the input dtype (:201), then qw_moe_balance.  With cdt == flat.dtype
    these are the stages and arguments of qw_moe_forward, so the output is
    identical; with cdt != flat.dtype (bf16 autocast on an fp32 stream) the
    rows are bf16 and the weighted sum fp32, as under the reference's autocast.
    save: keep the activations a backward pass reads (qw_moe_experts_save):
    gate, up, hidden [R, d_ff]; the unweighted expert rows are `y` itself.
    loop: the experts run one call per expert with rows (the reference's loop
    executor, :203-209), after reading the kept counts back to the host as the
    reference does.  profile: a list of per-expert seconds; each expert call is
    then bracketed by synchronisations and its wall time added to the list
    (the reference's profile_experts, src/quantweave_moe_model.py:220-233).
    static: the combine of the static dispatch, qw_moe_combine_static
    (`_static_output`, :235-245; the caller passes a capacity-free plan)."""
    dev = flat.device
    T, D = flat.shape
    E, K = moe.num_experts, moe.top_k
    R = T * K
    F_ = moe.experts[0].gate.out_features
    act_in = _hip.act_code(flat, "TopKMoE.forward")
    act = _hip.act_code(torch.empty(0, dtype=cdt), "TopKMoE.forward")
    mixed = act != act_in
    rw = _router_operand(router_w)
    i32 = dict(dtype=torch.int32, device=dev)
    r = dict(out=torch.empty_like(flat), probs=torch.empty(T, E, dtype=torch.float32, device=dev),
             top_idx=torch.empty(T, K, **i32), top_w=torch.empty(T, K, dtype=torch.float32, device=dev),
             counts=torch.empty(E, **i32), kept_counts=torch.empty(E, **i32), kept_offsets=torch.zeros(E + 1, **i32),
             slot_token=torch.empty(max(R, 1), **i32), route_slot=torch.empty(max(R, 1), **i32),
             slot_weight=torch.empty(max(R, 1), dtype=torch.float32, device=dev),
             dropped_token=torch.empty(max(R, 1), **i32), dropped_expert=torch.empty(max(R, 1), **i32),
             totals=torch.zeros(2, **i32), balance=torch.zeros((), dtype=torch.float32, device=dev))
    if not T:
        return r
    lib = _lib.load()
    s = _hip.stream(dev)
    p = {k: _hip.ptr(v) for k, v in r.items()}
    logits = torch.empty(T, E, dtype=torch.float32, device=dev)
    nb = lib.qw_moe_route_workspace_bytes(T, D, E)
    ws = _hip.workspace(nb, dev)
    _lib.call("qw_moe_route", _hip.ptr(flat), act_in, D, _hip.ptr(rw), _hip.act_code(rw, "router"), T, D, E, K,
              float(moe.router_temperature), _hip.ptr(bias), _hip.ptr(logits), p["probs"], p["top_idx"], p["top_w"],
              _hip.ptr(ws), nb, s)
    nb = lib.qw_moe_plan_workspace_bytes(T, K, E)
    ws = _hip.workspace(nb, dev)
    _lib.call("qw_moe_plan", p["top_idx"], p["top_w"], T, K, E, cap, p["counts"], p["kept_counts"],
              p["kept_offsets"], p["slot_token"], p["slot_weight"], p["route_slot"], p["dropped_token"],
              p["dropped_expert"], p["totals"], _hip.ptr(ws), nb, s)
    xc = flat.to(cdt) if mixed else flat
    max_rows = min(R, cap * E)
    y = torch.empty(R, D, dtype=cdt, device=dev)
    if save:
        for name in ("gate", "up", "hidden"):
            r[name] = torch.empty(R, F_, dtype=cdt, device=dev)
        r["y_unweighted"] = y  # the rows carry no route weight: the combine applies it
    nb = lib.qw_moe_experts_workspace_bytes(R if loop else max_rows, E, D, F_, act)
    ws = _hip.workspace(nb, dev)
    saved = [_hip.ptr(r[n]) for n in ("gate", "up", "hidden")] + [_hip.ptr(y)] if save else []
    fn = "qw_moe_experts_save" if save else "qw_moe_experts"
    if loop:
        import time

        kept = r["kept_counts"].tolist()  # host sync, as the reference's loop makes
        weights = pack.for_act(act)
        for e in range(E):
            if not kept[e]:
                continue
            offs = ctypes.c_void_p(r["kept_offsets"].data_ptr() + 4 * e)
            if profile is not None:
                torch.cuda.synchronize(dev)
                started = time.perf_counter()
            _lib.call(fn, _hip.ptr(xc), act, p["slot_token"], offs, 1, D, F_, R, min(cap, R),
                      *weights.expert_args(e), None, _hip.ptr(y), *saved, _hip.ptr(ws), nb, s)
            if profile is not None:
                torch.cuda.synchronize(dev)
                profile[e] += time.perf_counter() - started
    else:
        _lib.call(fn, _hip.ptr(xc), act, p["slot_token"], p["kept_offsets"], E, D, F_, max_rows, min(cap, R),
                  *pack.args_for(act), None, _hip.ptr(y), *saved, _hip.ptr(ws), nb, s)
    _lib.call("qw_moe_combine_static" if static else "qw_moe_combine_weighted", _hip.ptr(y), act, p["route_slot"],
              p["top_idx"], p["top_w"], T, K, D, p["out"], act_in, s)
    importance = torch.empty(E, dtype=torch.float32, device=dev)
    nb = lib.qw_moe_balance_workspace_bytes(T, E)
    ws = _hip.workspace(nb, dev)
    _lib.call("qw_moe_balance_ws", p["probs"], p["counts"], T, K, E, _hip.ptr(importance), p["balance"], _hip.ptr(ws),
              nb, s)
    return r


class _MoELayer(torch.autograd.Function):
    """TopKMoE.forward with gradients for the input, the router and the
    experts (src/quantweave_moe_model.py:113-164, :190-202 through autograd).

    Forward: ``_layer_chain`` (the inference kernels, one C call per stage),
    its expert call keeping the gate/up projections, the SiLU product and the
    unweighted expert rows (qw_moe_experts_save).  Backward:
      qw_moe_combine_backward   d(expert rows), d(router weights)
      grouped backward kernels  down, SwiGLU, gate and up
      qw_moe_combine_weighted   index_add of the row gradients (weights off)
      qw_moe_route_backward     renormalise + balance + softmax backward
    and the router's two plain products (library GEMMs)."""

    @staticmethod
    def forward(ctx, flat, router_w, moe, pack, cap, bias, cdt, loop, static, *weights):
        ctx.set_materialize_grads(False)
        flat = flat.detach().contiguous()
        r = _layer_chain(flat, cdt, router_w.detach(), moe, pack, cap, bias, save=flat.size(0) > 0, loop=loop,
                         static=static)
        saved = [r.get(n) for n in ("gate", "up", "hidden", "y_unweighted")]
        ctx.save_for_backward(flat, _router_operand(router_w), r["probs"], r["top_idx"], r["top_w"], r["counts"],
                              r["kept_offsets"], r["slot_token"], r["route_slot"], r["totals"], *saved)
        ctx.moe, ctx.pack, ctx.cap, ctx.cdt, ctx.router_dtype = moe, pack, cap, cdt, router_w.dtype
        ctx.mark_non_differentiable(r["top_idx"], r["top_w"], r["counts"], r["kept_counts"], r["totals"],
                                    r["dropped_token"], r["dropped_expert"])
        return (r["out"], r["probs"], r["balance"], r["top_idx"], r["top_w"], r["counts"], r["kept_counts"],
                r["totals"], r["dropped_token"], r["dropped_expert"])

    @staticmethod
    def backward(ctx, d_out, d_probs, d_balance, *unused):
        (flat, rw, probs, top_idx, top_w, counts, kept_offsets, slot_token, route_slot, totals, g, u, h,
         y) = ctx.saved_tensors
        moe, cdt = ctx.moe, ctx.cdt
        n_w = 3 * len(moe.experts)
        need_x, need_router = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        need_experts = any(ctx.needs_input_grad[9:9 + n_w])
        T, D = flat.shape
        E, K = moe.num_experts, moe.top_k
        R = T * K
        dev = flat.device
        s = _hip.stream(dev)
        act_in = _hip.act_code(flat, "TopKMoE.backward")
        act = _hip.act_code(torch.empty(0, dtype=cdt), "TopKMoE.backward")
        d_flat = None
        expert_grads = [None] * n_w
        d_top_w = torch.zeros(T, K, dtype=torch.float32, device=dev)
        if T and d_out is not None and (need_x or need_router or need_experts):
            from .moe_kernels import _backward

            d_out = d_out.contiguous().to(flat.dtype)
            dy = torch.empty_like(y)
            _lib.call("qw_moe_combine_backward", _hip.ptr(d_out), act_in, _hip.ptr(y), act, _hip.ptr(route_slot),
                      _hip.ptr(top_w), T, K, D, _hip.ptr(dy), _hip.ptr(d_top_w), s)
            if need_x or need_experts:
                stacks = ctx.pack.plain(moe.experts, cdt)
                plan = _RowPlan(kept_offsets, E, min(ctx.cap, R))
                xp = torch.empty(R, D, dtype=cdt, device=dev)
                _lib.call("qw_moe_permute", _hip.ptr(flat.to(cdt)), act, D, _hip.ptr(slot_token), _hip.ptr(totals), R,
                          _hip.ptr(xp), s)
                wdt = moe.experts[0].gate.weight.dtype  # fp32 parameters: unrounded fp32 gradients
                gwd = torch.float32 if wdt == torch.float32 else None
                dh, d_down = _backward(dy, h, stacks[2], plan, act, True, need_experts, grad_w_dtype=gwd)
                dg, du = torch.empty_like(g), torch.empty_like(u)
                _lib.call("qw_swiglu_backward", _hip.ptr(dh), _hip.ptr(g), _hip.ptr(u), act, g.numel(), _hip.ptr(dg),
                          _hip.ptr(du), s)
                dxp, d_gate = _backward(dg, xp, stacks[0], plan, act, need_x, need_experts, grad_w_dtype=gwd)
                dxp, d_up = _backward(du, xp, stacks[1], plan, act, need_x, need_experts, grad_x=dxp,
                                      grad_w_dtype=gwd)
                if need_experts:
                    for j, (n, gw) in enumerate((("gate", d_gate), ("up", d_up), ("down", d_down))):
                        per = gw.to(getattr(moe.experts[0], n).weight.dtype).unbind(0)
                        for i in range(len(moe.experts)):
                            expert_grads[3 * i + j] = per[i]
                if need_x:
                    d_flat = torch.empty_like(flat)
                    _lib.call("qw_moe_combine_weighted", _hip.ptr(dxp), act, _hip.ptr(route_slot), _hip.ptr(top_idx),
                              None, T, K, D, _hip.ptr(d_flat), act_in, s)
        d_router = None
        if T and (need_x or need_router) and (d_out is not None or d_probs is not None or d_balance is not None):
            d_scores = torch.empty(T, E, dtype=torch.float32, device=dev)
            gp = None if d_probs is None else d_probs.contiguous().float()
            gb = None if d_balance is None else d_balance.reshape(1).contiguous().float()
            _lib.call("qw_moe_route_backward", _hip.ptr(probs), _hip.ptr(top_idx), _hip.ptr(top_w), _hip.ptr(d_top_w),
                      _hip.ptr(gp), _hip.ptr(gb), _hip.ptr(counts), T, E, K, float(moe.router_temperature),
                      _hip.ptr(d_scores), s)
            if need_router:
                d_router = (d_scores.t() @ flat.float()).to(ctx.router_dtype)
            if need_x:
                dx_router = (d_scores @ rw.float()).to(flat.dtype)
                d_flat = dx_router if d_flat is None else d_flat + dx_router
        return (d_flat, d_router, None, None, None, None, None, None, None, *expert_grads)


class _RowPlan:
    """Device row offsets of the plan-ordered rows, in the shape the grouped
    matmul helpers take (offsets, experts, per-expert row bound)."""

    def __init__(self, offsets: Tensor, experts: int, max_count: int) -> None:
        self.offsets = offsets
        self.num_experts = experts
        self.max_count = max_count


def set_moe_kernel(model: nn.Module, kernel: str) -> str:
    """Expert executor of every TopKMoE in `model`: "loop", "triton" (the
    grouped kernels; "hip" is an alias) or "auto".  Returns the active one,
    with the reference's names and errors (src/quantweave_moe_model.py:381-393):
    "auto" gives "triton" where the grouped kernels can run and "loop"
    elsewhere; asking for "triton" (or "hip") where they cannot raises.

    Both executors run the same HIP kernels: "triton" launches all experts at
    once, "loop" one launch per expert with rows after reading the kept counts
    back to the host (the reference's per-expert loop, :203-209)."""
    if kernel not in {"loop", "triton", "auto", "hip"}:
        raise ValueError("kernel must be loop, triton or auto")
    from .moe_kernels import kernels_available

    available = kernels_available(next(model.parameters()).device)
    if kernel in ("triton", "hip") and not available:
        raise RuntimeError("the grouped MoE kernels need a CUDA (ROCm) device and the built libqwmoe.so")
    grouped = kernel in ("triton", "hip") or (kernel == "auto" and available)
    for m in model.modules():
        if isinstance(m, TopKMoE):
            m.use_triton_kernels = grouped
    if not grouped:
        return "loop"
    return "hip" if kernel == "hip" else "triton"
