"""Calibrate the router logit-bias scale tau of the synthetic Zipf(1.1) workload.

The synthetic router adds b[perm[i]] = tau * ln(p_i), p_i proportional to i^-1.1, to the logits
x . W_r^T (x ~ N(0,1) bf16, W_r ~ N(0, 0.02) bf16, hidden 2048). tau is chosen so that the
realised per-expert top-8 selection frequencies over 65536 tokens, sorted in decreasing order,
best fit Zipf(1.1) in L1 distance (the head saturates because 8 * p_1 > 1, so the fit is not
exact). Run: python -m mtp_amd.calibrate_zipf  (prints the best tau and the fit table).
"""

from __future__ import annotations

import numpy as np
import torch

from mtp_amd import synth


def selection_frequencies(logits: torch.Tensor, bias: torch.Tensor, k: int = 8) -> np.ndarray:
    ids = torch.topk(logits + bias, k, dim=-1).indices
    counts = torch.bincount(ids.reshape(-1), minlength=logits.shape[1]).double()
    return (counts / counts.sum()).numpy()


def calibrate(tokens: int = 65536, taus=None, seed_layer: int = 0) -> tuple[float, list]:
    E, H = synth.NUM_EXPERTS, synth.HIDDEN
    w = synth.make_router(E, H, seed=2000 + seed_layer).float()
    logits = torch.cat([synth.make_tokens(8192, H, seed=100 + c).float() @ w.T
                        for c in range(tokens // 8192)])
    ranks = np.arange(1, E + 1, dtype=np.float64)
    p = ranks ** -synth.ZIPF_S
    p /= p.sum()
    taus = taus if taus is not None else np.round(np.arange(0.05, 1.01, 0.05), 3)
    table = []
    for tau in taus:
        bias = synth.zipf_logit_bias(E, seed=3000 + seed_layer, tau=float(tau))
        f = np.sort(selection_frequencies(logits, bias))[::-1]
        table.append((float(tau), float(np.abs(f - p).sum()), int((f == 0).sum()), float(f[0]), float(f[-1])))
    best = min(table, key=lambda r: r[1])
    return best[0], table


if __name__ == "__main__":
    tau, table = calibrate()
    print("tau     L1(f_sorted, zipf)  zero-freq experts  f_max     f_min")
    for row in table:
        print(f"{row[0]:5.2f}   {row[1]:.4f}              {row[2]:4d}             {row[3]:.4f}   {row[4]:.2e}")
    print(f"best tau = {tau}")
