"""Thin helpers that call the C ABI with torch device tensors (tests only)."""

import numpy as np
import torch

from quantaweave_amd import _hip, _lib

P = _hip.ptr


def dev(a, dtype=None):
    t = torch.as_tensor(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda().contiguous()


def s():
    return _hip.stream(torch.device("cuda"))


def route_from_logits(logits: torch.Tensor, k: int, bias: torch.Tensor | None = None):
    T, E = logits.shape
    probs = torch.empty(T, E, dtype=torch.float32, device="cuda")
    idx = torch.empty(T, k, dtype=torch.int32, device="cuda")
    w = torch.empty(T, k, dtype=torch.float32, device="cuda")
    _lib.call("qw_moe_route_from_logits", P(logits), T, E, k, P(bias), P(probs), P(idx), P(w), s())
    torch.cuda.synchronize()
    return probs, idx, w


def route(x: torch.Tensor, router_w: torch.Tensor, k: int, temperature=1.0, bias=None):
    T, D = x.shape
    E = router_w.shape[0]
    logits = torch.empty(T, E, dtype=torch.float32, device="cuda")
    probs = torch.empty(T, E, dtype=torch.float32, device="cuda")
    idx = torch.empty(T, k, dtype=torch.int32, device="cuda")
    w = torch.empty(T, k, dtype=torch.float32, device="cuda")
    nb = _lib.load().qw_moe_route_workspace_bytes(T, D, E)
    ws = _hip.workspace(nb, torch.device("cuda"))
    _lib.call("qw_moe_route", P(x), _hip.act_code(x, "x"), x.stride(0), P(router_w), _hip.act_code(router_w, "w"), T,
              D, E, k, float(temperature), P(bias), P(logits), P(probs), P(idx), P(w), P(ws), nb, s())
    torch.cuda.synchronize()
    return logits, probs, idx, w


def plan(top_idx: torch.Tensor, top_w: torch.Tensor, E: int, cap: int):
    T, k = top_idx.shape
    R = T * k
    z = lambda n, dt=torch.int32: torch.full((max(n, 1),), -7, dtype=dt, device="cuda")  # noqa: E731
    out = dict(counts=z(E), kept_counts=z(E), kept_offsets=z(E + 1), slot_token=z(R),
               slot_weight=z(R, torch.float32), route_slot=z(R), dropped_token=z(R), dropped_expert=z(R),
               totals=z(2))
    nb = _lib.load().qw_moe_plan_workspace_bytes(T, k, E)
    ws = _hip.workspace(nb, torch.device("cuda"))
    _lib.call("qw_moe_plan", P(top_idx), P(top_w), T, k, E, cap, P(out["counts"]), P(out["kept_counts"]),
              P(out["kept_offsets"]), P(out["slot_token"]), P(out["slot_weight"]), P(out["route_slot"]),
              P(out["dropped_token"]), P(out["dropped_expert"]), P(out["totals"]), P(ws), nb, s())
    torch.cuda.synchronize()
    res = {k_: v.cpu().numpy() for k_, v in out.items()}
    kept, dropped = int(res["totals"][0]), int(res["totals"][1])
    res["slot_token"] = res["slot_token"][:kept]
    res["slot_weight"] = res["slot_weight"][:kept]
    res["dropped_token"] = res["dropped_token"][:dropped]
    res["dropped_expert"] = res["dropped_expert"][:dropped]
    res["route_slot"] = res["route_slot"][:R]
    return res


PATHS = {"auto": _lib.QW_PATH_AUTO, "generic": _lib.QW_PATH_GENERAL, "mfma": _lib.QW_PATH_MFMA,
         "stream": _lib.QW_PATH_STREAM}


def experts(x, offsets, fmt, gate, up, down, gate_s=None, up_s=None, down_s=None, group_in=0, group_ff=0,
            row_index=None, row_weight=None, max_rows=None, rows_per_expert=0, path="auto"):
    D = x.shape[1]
    E, F_ = gate.shape[0], gate.shape[1]
    rows = int(offsets[-1].item()) if max_rows is None else max_rows
    act = _hip.act_code(x, "x")
    y = torch.full((max(rows, 1), D), float("nan"), dtype=x.dtype, device="cuda")
    nb = _lib.load().qw_moe_experts_workspace_bytes(rows, E, D, F_, act)
    ws = _hip.workspace(nb, torch.device("cuda"))
    _lib.call("qw_moe_experts_on_path", PATHS[path], P(x), act, P(row_index), P(offsets), E, D, F_, rows,
              rows_per_expert, fmt, group_in, group_ff, P(gate), P(gate_s), P(up), P(up_s), P(down), P(down_s),
              P(row_weight), P(y), P(ws), nb, s())
    torch.cuda.synchronize()
    return y[:rows]
