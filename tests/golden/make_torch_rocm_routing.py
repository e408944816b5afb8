"""Record torch-ROCm's routing primitives on an MI355X as fixtures.

The reference routes with torch's GPU kernels (src/quantweave_moe_model.py:
127-136): softmax, topk, gather and a sum over the k chosen weights.  On the
device those have fixed bits that the oracle's CPU restatement follows (the
tie order of torch.topk and the summation order of w.sum(-1)).  This script
runs those torch calls on the GPU and stores inputs and outputs in
torch_rocm_routing.npz, which tests/test_oracle.py reads on the CPU.  It uses
torch only (no reference code):

    python tests/golden/make_torch_rocm_routing.py [--out PATH]
"""

import argparse
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "torch_rocm_routing.npz"
TIE_KS = (1, 2, 3, 4, 5, 6, 7, 8, 16, 31, 32, 33, 40)
SUM_KS = tuple(range(1, 17)) + (31, 32, 33, 63, 64, 65, 100, 127)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", type=Path, default=OUT)
    dest = ap.parse_args().out
    assert torch.cuda.is_available(), "run on the GPU"
    dev = "cuda"
    rng = np.random.RandomState(20260)
    out = {"torch_version": np.array(torch.__version__), "hip_version": np.array(str(torch.version.hip))}
    # probabilities on a coarse grid: many exact ties, at the top and at the k-th place
    for E in (64, 184):
        P = (rng.randint(1, 9, size=(400, E)) / 16.0).astype(np.float32)
        P[0] = 0.25
        P[1] = 0.0625
        P[1, [3, 40, E - 1]] = 0.5
        out[f"ties_E{E}_p"] = P
        for k in TIE_KS:
            v, i = torch.from_numpy(P).to(dev).topk(k, dim=-1)
            out[f"ties_E{E}_k{k}_idx"] = i.cpu().numpy().astype(np.int32)
    # biased scores (logits + bias) that tie; the chosen indices only
    L = (np.rint(rng.randn(300, 64) * 2) / 2).astype(np.float32)
    b = (np.rint(rng.randn(64) * 2) / 4).astype(np.float32)
    out["biased_logits"], out["biased_bias"] = L, b
    for k in (2, 3, 4, 8):
        i = (torch.from_numpy(L).to(dev) + torch.from_numpy(b).to(dev)).topk(k, dim=-1).indices
        out[f"biased_k{k}_idx"] = i.cpu().numpy().astype(np.int32)
    # the renormalising sum over k chosen weights
    for k in SUM_KS:
        w = rng.rand(256, k).astype(np.float32)
        out[f"sum_k{k}_w"] = w
        out[f"sum_k{k}_s"] = torch.from_numpy(w).to(dev).sum(dim=-1).cpu().numpy()
    # softmax rows (the oracle's own exp is compared within a few ulp)
    for E in (8, 64, 184):
        Ls = (rng.randn(256, E) * 2).astype(np.float32)
        out[f"softmax_E{E}_logits"] = Ls
        out[f"softmax_E{E}_probs"] = torch.from_numpy(Ls).to(dev).softmax(dim=-1).cpu().numpy()
    np.savez_compressed(dest, **out)
    print(f"wrote {dest} ({dest.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
