"""CPU oracle for the routed MoE expert-FFN forward — TEST INFRASTRUCTURE ONLY.

The GPU parity tests compare against it.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the CPU-baseline leg of ``bench.py`` import it; the product library
(``quantaweave_amd``) never does.

Two layers:

* ``qw_oracle.c`` (built to ``liboracle.so`` with gcc, ctypes-loaded): the
  bit-exact parts — deterministic softmax/top-k/renormalisation, capacity and
  the capacity plan, int8/int4 quantisation and dequantisation.
* numpy (this file): the floating-point expert FFN and the combine, following
  the reference's rounding points, in float64 with explicit rounding to the
  activation dtype.

Reference lines each function restates are given in its docstring (paths are
relative to the QuantaWeave source tree).
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "qw_oracle.c"
LIB = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    """Compile the C restatement (gcc, IEEE single precision, no contraction)."""
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
           "-o", str(LIB), str(SRC), "-lm"]
    subprocess.run(cmd, check=True)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists() or LIB.stat().st_mtime < SRC.stat().st_mtime:
            build()
        L = ctypes.CDLL(str(LIB))
        P = ctypes.c_void_p
        i32, i64, f32, f64 = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_double
        L.orc_expf.argtypes, L.orc_expf.restype = [f32], f32
        L.orc_softmax_row.argtypes = [P, i32, P]
        L.orc_route_from_logits.argtypes = [P, i32, i32, i32, P, P, P, P]
        L.orc_route_select.argtypes = [P, i32, i32, i32, P, i32, P, P, P]
        L.orc_route_select_probs.argtypes = [P, P, i32, i32, i32, P, i32, P, P]
        L.orc_topk_weight_sum.argtypes, L.orc_topk_weight_sum.restype = [P, i32], f32
        L.orc_router_logits.argtypes = [P, P, i32, i32, i32, f32, P]
        L.orc_capacity.argtypes, L.orc_capacity.restype = [i64, i64, i64, f64, f64, i64, i32], i64
        L.orc_plan.argtypes = [P, P, i32, i32, i32, i64, P, P, P, P, P, P, P, P, P]
        L.orc_plan.restype = i32
        L.orc_quantize.argtypes = [P, i64, i64, i32, i64, P, P]
        L.orc_dequantize.argtypes = [P, P, i32, i64, i64, i64, P]
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------------------
# bf16 helpers (round to nearest even, as torch's .to(torch.bfloat16))
# ---------------------------------------------------------------------------
def round_bf16(a: np.ndarray) -> np.ndarray:
    """float32 array rounded to the nearest bf16 value (returned as float32)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = u.astype(np.uint32).view(np.float32)
    out = np.where(nan, a, out)
    return out


def round_f16(a: np.ndarray) -> np.ndarray:
    """float32 array rounded to the nearest IEEE binary16 value (returned as
    float32): numpy's conversion rounds to nearest even and overflows to
    infinity, as torch's .to(torch.float16) does."""
    with np.errstate(over="ignore"):
        return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_act(a: np.ndarray, dtype: str) -> np.ndarray:
    a = np.asarray(a, dtype=np.float32)
    if dtype == "bf16":
        return round_bf16(a)
    if dtype == "f16":
        return round_f16(a)
    return a


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """uint16 bit patterns of bf16-representable float32 values."""
    return (round_bf16(a).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------
# routing
# ---------------------------------------------------------------------------
def expf(x: float) -> float:
    return lib().orc_expf(float(x))


def softmax(logits: np.ndarray) -> np.ndarray:
    """Row softmax with the exactly specified exp and summation order."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    out = np.empty_like(logits)
    for t in range(T):
        lib().orc_softmax_row(_ptr(logits[t]), E, _ptr(out[t]))
    return out


def router_logits(x: np.ndarray, w: np.ndarray, temperature: float = 1.0) -> np.ndarray:
    """src/quantweave_moe_model.py:128 — fp32 logits (double accumulation)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    T, D = x.shape
    E = w.shape[0]
    out = np.empty((T, E), dtype=np.float32)
    lib().orc_router_logits(_ptr(x), _ptr(w), T, D, E, float(temperature), _ptr(out))
    return out


def route_from_logits(logits: np.ndarray, top_k: int, expert_bias: np.ndarray | None = None,
                      select: str = "probs"):
    """src/quantweave_moe_model.py:129-137.  Returns (probs, top_idx int32, top_w).

    select="logits" is the decode step's selection (src/fast_decode.py:172):
    top-k of the scores (plus the bias, if any) rather than of the
    probabilities; it differs only where rounded probabilities tie."""
    if select not in ("probs", "logits"):
        raise ValueError("select must be 'probs' or 'logits'")
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    probs = np.empty((T, E), dtype=np.float32)
    idx = np.empty((T, top_k), dtype=np.int32)
    w = np.empty((T, top_k), dtype=np.float32)
    bias = None if expert_bias is None else np.ascontiguousarray(expert_bias, dtype=np.float32)
    lib().orc_route_select(_ptr(logits), T, E, top_k, _ptr(bias), int(select == "logits"), _ptr(probs), _ptr(idx),
                           _ptr(w))
    return probs, idx, w


def route_from_probs(logits: np.ndarray, probs: np.ndarray, top_k: int, expert_bias: np.ndarray | None = None,
                     select: str = "probs"):
    """The selection and renormalisation of route_from_logits from given
    probabilities (e.g. torch's softmax on the device).  Returns (top_idx
    int32, top_w)."""
    if select not in ("probs", "logits"):
        raise ValueError("select must be 'probs' or 'logits'")
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    probs = np.ascontiguousarray(probs, dtype=np.float32)
    T, E = logits.shape
    assert probs.shape == (T, E)
    idx = np.empty((T, top_k), dtype=np.int32)
    w = np.empty((T, top_k), dtype=np.float32)
    bias = None if expert_bias is None else np.ascontiguousarray(expert_bias, dtype=np.float32)
    lib().orc_route_select_probs(_ptr(logits), _ptr(probs), T, E, top_k, _ptr(bias), int(select == "logits"),
                                 _ptr(idx), _ptr(w))
    return idx, w


def topk_weight_sum(w: np.ndarray) -> np.ndarray:
    """Per-row sum of a [T, k] array in torch-ROCm's reduction order (k < 128)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    return np.array([lib().orc_topk_weight_sum(_ptr(row), w.shape[1]) for row in w], dtype=np.float32)


def capacity(tokens: int, top_k: int, experts: int, capacity_factor: float, capacity_scale: float = 1.0,
             min_capacity: int = 4, drop_overflow: bool = True) -> int:
    """src/quantweave_moe_model.py:100-111."""
    return int(lib().orc_capacity(tokens, top_k, experts, capacity_factor, capacity_scale, min_capacity,
                                  int(bool(drop_overflow))))


def plan(top_idx: np.ndarray, top_w: np.ndarray, experts: int, cap: int) -> dict:
    """src/quantweave_moe_model.py:166-188 — one stable sort by (expert, -weight, route)."""
    top_idx = np.ascontiguousarray(top_idx, dtype=np.int32)
    top_w = np.ascontiguousarray(top_w, dtype=np.float32)
    T, K = top_idx.shape
    R = T * K
    out = dict(
        counts=np.zeros(experts, np.int32), kept_counts=np.zeros(experts, np.int32),
        kept_offsets=np.zeros(experts + 1, np.int32), slot_token=np.zeros(R, np.int32),
        slot_weight=np.zeros(R, np.float32), route_slot=np.zeros(R, np.int32),
        dropped_token=np.zeros(R, np.int32), dropped_expert=np.zeros(R, np.int32), totals=np.zeros(2, np.int32),
    )
    lib().orc_plan(_ptr(top_idx), _ptr(top_w), T, K, experts, int(cap), *(_ptr(out[k]) for k in (
        "counts", "kept_counts", "kept_offsets", "slot_token", "slot_weight", "route_slot", "dropped_token",
        "dropped_expert", "totals")))
    kept, dropped = int(out["totals"][0]), int(out["totals"][1])
    out["slot_token"] = out["slot_token"][:kept]
    out["slot_weight"] = out["slot_weight"][:kept]
    out["dropped_token"] = out["dropped_token"][:dropped]
    out["dropped_expert"] = out["dropped_expert"][:dropped]
    return out


# ---------------------------------------------------------------------------
# QW_BF16T weight tiles (a layout of this library, not of the reference)
# ---------------------------------------------------------------------------
def _tile_perm(shape):
    E, R, K = shape
    if R % 8 or K % 64:
        raise ValueError("tiles need out % 8 == 0 and in % 64 == 0")
    rb = np.arange(R // 8)[:, None, None]
    r = np.arange(8)[None, :, None]
    phys = np.arange(8)[None, None, :]
    return (R, K), rb, r, phys ^ (((8 * rb + r) >> 1) & 7)


def tile_bf16(w: np.ndarray) -> np.ndarray:
    """[E, out, in] -> the same values in QW_BF16T order (tile (rb, kb) = 512
    consecutive elements; its 16-byte piece 8*r + phys holds row 8*rb + r,
    columns 64*kb + 8*p .. +7 with p = phys ^ (((8*rb + r) >> 1) & 7))."""
    E = w.shape[0]
    (R, K), rb, r, p = _tile_perm(w.shape)
    w6 = w.reshape(E, R // 8, 8, K // 64, 8, 8).transpose(0, 3, 1, 2, 4, 5)  # E, kb, rb, r, p, 8
    t = w6[:, :, rb, r, p, :]  # E, kb, rb, r, phys, 8
    return np.ascontiguousarray(t.transpose(0, 2, 1, 3, 4, 5)).reshape(E, R, K)


def untile_bf16(t: np.ndarray) -> np.ndarray:
    """Inverse of tile_bf16."""
    E = t.shape[0]
    (R, K), rb, r, p = _tile_perm(t.shape)
    t6 = t.reshape(E, R // 8, K // 64, 8, 8, 8).transpose(0, 2, 1, 3, 4, 5)  # E, kb, rb, r, phys, 8
    w6 = np.empty_like(t6)  # E, kb, rb, r, p, 8
    w6[:, :, rb, r, p, :] = t6
    return np.ascontiguousarray(w6.transpose(0, 2, 3, 1, 4, 5)).reshape(E, R, K)


# ---------------------------------------------------------------------------
# quantisation
# ---------------------------------------------------------------------------
def quant_geometry(in_features: int, bits: int, group_size: int | None):
    """src/quantization.py:32-38: (group, padded, groups, stored columns)."""
    group = group_size or (in_features if bits == 8 else 32)
    padded = -(-in_features // group) * group
    return group, padded, padded // group, (padded if bits == 8 else padded // 2)


def quantize(w: np.ndarray, bits: int, group_size: int | None = None):
    """src/quantization.py:43-59.  Returns (qweight, scales, group)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    group, padded, groups, stored = quant_geometry(cols, bits, group_size)
    q = np.zeros((rows, stored), dtype=np.int8 if bits == 8 else np.uint8)
    s = np.zeros((rows, groups), dtype=np.float32)
    lib().orc_quantize(_ptr(w), rows, cols, bits, group, _ptr(q), _ptr(s))
    return q, s, group


def dequantize(qweight: np.ndarray, scales: np.ndarray, bits: int, in_features: int, group: int) -> np.ndarray:
    """src/quantization.py:61-69: fp32 [out, in]."""
    qweight = np.ascontiguousarray(qweight)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    rows = qweight.shape[0]
    out = np.empty((rows, in_features), dtype=np.float32)
    lib().orc_dequantize(_ptr(qweight), _ptr(scales), bits, rows, in_features, group, _ptr(out))
    return out


# ---------------------------------------------------------------------------
# expert FFN and combine (floating point, numpy)
# ---------------------------------------------------------------------------
def _silu(g: np.ndarray) -> np.ndarray:
    g64 = g.astype(np.float64)
    return (g64 / (1.0 + np.exp(-g64))).astype(np.float32)


def linear(x: np.ndarray, w: np.ndarray, dtype: str, accum: str = "f64") -> np.ndarray:
    """F.linear(x, w) in `dtype`: products/accumulation in float64 (or float32
    with accum="f32", the speed mode of the CPU baseline), one rounding to
    float32 and then to the activation dtype."""
    if accum == "f32":
        out = np.asarray(x, np.float32) @ np.asarray(w, np.float32).T
    else:
        out = (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)
    return round_act(out, dtype)


def swiglu(x: np.ndarray, gate: np.ndarray, up: np.ndarray, down: np.ndarray, dtype: str,
           accum: str = "f64") -> np.ndarray:
    """SparseSwiGLU.forward, src/quantweave_moe_model.py:59-60, with the
    reference's rounding points: gate/up outputs, silu, the product and the
    down output are each rounded to `dtype`."""
    g = linear(x, gate, dtype, accum)
    u = linear(x, up, dtype, accum)
    h = round_act(round_act(_silu(g), dtype) * u, dtype)
    return linear(h, down, dtype, accum)


def _codes_times_scales(q: np.ndarray, scales: np.ndarray, bits: int, in_features: int, group: int) -> np.ndarray:
    """q * scale per group in float64 (exact: a code has at most 8 bits, a
    scale 24), from the stored bytes (the layout of src/quantization.py:43-59)."""
    q = np.asarray(q)
    if bits == 4:
        u = q.astype(np.int16)
        codes = np.empty((q.shape[0], q.shape[1] * 2), np.int16)
        codes[:, 0::2] = (u & 0xF) - 8
        codes[:, 1::2] = (u >> 4) - 8
    else:
        codes = q.astype(np.int16)
    s = np.repeat(np.asarray(scales, np.float64), group, axis=1)
    return (codes.astype(np.float64) * s)[:, :in_features]


def expert_weights(w: dict, e: int, dtype: str, quantised: str = "reference") -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Effective (gate, up, down) of expert e as the reference multiplies them:
    float weights as stored; quantised ones dequantised (fp32) and cast to the
    activation dtype (src/quantization.py:72).  quantised="exact" instead keeps
    q * scale unrounded (float64): the arithmetic of the weight-streaming
    decode kernels, which multiply the exact codes and apply each group's fp32
    scale to the group's partial sum."""
    if w["format"] in ("f32", "bf16", "f16"):
        # float weights are cast to the activation dtype (src/moe_kernels.py:191-193)
        return tuple(round_act(w[n][e], dtype) for n in ("gate", "up", "down"))
    bits = 8 if w["format"] == "i8" else 4
    d, f = w["d_model"], w["d_ff"]
    if quantised == "exact":
        return (_codes_times_scales(w["gate"][e], w["gate_scales"][e], bits, d, w["group_in"]),
                _codes_times_scales(w["up"][e], w["up_scales"][e], bits, d, w["group_in"]),
                _codes_times_scales(w["down"][e], w["down_scales"][e], bits, f, w["group_ff"]))
    g = dequantize(w["gate"][e], w["gate_scales"][e], bits, d, w["group_in"])
    u = dequantize(w["up"][e], w["up_scales"][e], bits, d, w["group_in"])
    dn = dequantize(w["down"][e], w["down_scales"][e], bits, f, w["group_ff"])
    return round_act(g, dtype), round_act(u, dtype), round_act(dn, dtype)


def experts_forward(x_rows: np.ndarray, kept_counts: np.ndarray, w: dict, dtype: str, accum: str = "f64",
                    quantised: str = "reference") -> np.ndarray:
    """The per-expert loop, src/quantweave_moe_model.py:203-209: expert e runs on
    its contiguous block of plan-ordered rows (quantised weights as
    expert_weights gives them)."""
    out = np.zeros((x_rows.shape[0], w["d_model"]), dtype=np.float32)
    start = 0
    for e, c in enumerate(kept_counts.tolist()):
        if c:
            g, u, dn = expert_weights(w, e, dtype, quantised)
            out[start:start + c] = swiglu(x_rows[start:start + c], g, u, dn, dtype, accum)
        start += c
    return out


def combine(y_rows: np.ndarray, slot_token: np.ndarray, slot_weight: np.ndarray, tokens: int, dtype: str) -> np.ndarray:
    """src/quantweave_moe_model.py:192, :210-211: `(Y * weights[:, None])` in
    fp32, `.to(dtype)`, then `zeros.index_add_(0, tokens, ...)`: torch adds
    the rows into a float32 accumulator in the order of `tokens` (plan order)
    and rounds to `dtype` once at the end (what its CPU kernel does for a
    bf16 output; identical to a rounding per add when a token has at most two
    routes)."""
    contrib = round_act(y_rows.astype(np.float32) * slot_weight[:, None].astype(np.float32), dtype)
    acc = np.zeros((tokens, y_rows.shape[1]), dtype=np.float32)
    for s, t in enumerate(slot_token.tolist()):
        acc[t] = acc[t] + contrib[s]
    return round_act(acc, dtype)


def combine_static(y_rows: np.ndarray, slot_token: np.ndarray, slot_weight: np.ndarray, tokens: int,
                   dtype: str) -> np.ndarray:
    """src/quantweave_moe_model.py:235-245 (TopKMoE._static_output): the dense
    weights cast to `dtype` before the product, `output = output + term`
    rounded to `dtype` after every add, experts in ascending order (the plan
    order of a token's routes; experts it does not use add exact zeros)."""
    w = round_act(np.asarray(slot_weight, np.float32), dtype)
    contrib = round_act(y_rows.astype(np.float32) * w[:, None], dtype)
    out = np.zeros((tokens, y_rows.shape[1]), dtype=np.float32)
    for s, t in enumerate(slot_token.tolist()):
        out[t] = round_act(out[t] + contrib[s], dtype)
    return out


def decode_step(x: np.ndarray, router_w: np.ndarray, w: dict, *, top_k: int, dtype: str, temperature: float = 1.0,
                expert_bias: np.ndarray | None = None, residual: np.ndarray | None = None,
                logits: np.ndarray | None = None, accum: str = "f64", probs: np.ndarray | None = None):
    """The routed-expert lines of FastDecoder._step, src/fast_decode.py:170-177.

    x [T, d] fp32 (the normed hidden state), router_w fp32 [E, d].  Routing in
    fp32 with selection on the scores (:171-174); every route is evaluated (no
    capacity); expert inputs are x rounded to `dtype` (:174); each expert's
    SwiGLU in `dtype` (:175-177, the weights as `expert_weights` gives them);
    then out = residual + sum_j float(y_j) * w_j in fp32, in top-k order.
    `probs`, when given, is the softmax of `logits` as computed elsewhere (torch
    on the device); the selection then starts from it.
    Returns a dict with logits, probs, top_idx, top_w, y [T, k, d] and out."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, d = x.shape
    if logits is None:
        logits = router_logits(x, router_w, temperature)
    if probs is None:
        probs, idx, tw = route_from_logits(logits, top_k, expert_bias, select="logits")
    else:
        idx, tw = route_from_probs(logits, probs, top_k, expert_bias, select="logits")
    xc = round_act(x, dtype)
    y = np.zeros((T, top_k, d), dtype=np.float32)
    for e in np.unique(idx).tolist():
        tok, j = np.nonzero(idx == e)
        g, u, dn = expert_weights(w, e, dtype)
        y[tok, j] = swiglu(xc[tok], g, u, dn, dtype, accum)
    acc = np.zeros((T, d), dtype=np.float32)
    for j in range(top_k):
        acc = (acc + y[:, j] * tw[:, j:j + 1]).astype(np.float32)
    out = acc if residual is None else (np.asarray(residual, np.float32) + acc).astype(np.float32)
    return dict(logits=logits, probs=probs, top_idx=idx, top_w=tw, y=y, out=out)


def moe_forward(x: np.ndarray, router_w: np.ndarray, w: dict, *, top_k: int, cap: int, dtype: str,
                temperature: float = 1.0, expert_bias: np.ndarray | None = None, logits: np.ndarray | None = None,
                accum: str = "f64", probs: np.ndarray | None = None):
    """TopKMoE.forward, src/quantweave_moe_model.py:113-164 (dynamic dispatch).

    x [T, d] holds activation values (already rounded to `dtype`).  Returns a
    dict with the routing, the plan and the output [T, d] (float32 values
    representable in `dtype`).
    """
    T = x.shape[0]
    E = router_w.shape[0]
    if logits is None:
        logits = router_logits(x, router_w, temperature)
    if probs is None:
        probs, idx, tw = route_from_logits(logits, top_k, expert_bias)
    else:
        idx, tw = route_from_probs(logits, probs, top_k, expert_bias)
    p = plan(idx, tw, E, cap)
    rows = x[p["slot_token"]]
    y = experts_forward(rows, p["kept_counts"], w, dtype, accum)
    out = combine(y, p["slot_token"], p["slot_weight"], T, dtype)
    importance = probs.astype(np.float64).mean(axis=0)
    assignments = np.bincount(idx.reshape(-1), minlength=E) / float(T * top_k)
    balance = float(E * (importance * assignments).sum())
    return dict(logits=logits, probs=probs, top_idx=idx, top_w=tw, plan=p, y=y, out=out, balance=balance)
