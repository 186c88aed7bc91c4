"""Parity helpers shared by the GPU tests, smoke() and bench.py.

Acceptance rule, applied per layer call:
  * spikes bit-exact, except for at most floor(1e-4 * n_neuron_steps) mismatches, each of
    which must have a reference membrane within 1e-3 of V_th;
  * charged membranes within 1e-3 * max(|v_ref|, V_th), compared wherever the spike
    history of the neuron agrees with the reference up to the previous step (after an
    allowed near-threshold flip the two trajectories legitimately diverge).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

SPIKE_FLIP_FRACTION = 1e-4
NEAR_THRESHOLD = 1e-3
MEMBRANE_RTOL = 1e-3


@dataclass
class ParityReport:
    n: int                 # neuron-steps compared
    spike_mismatch: int
    far_mismatch: int      # mismatches whose reference membrane is not near threshold
    membrane_max_rel: float
    membrane_compared: int

    @property
    def ok(self) -> bool:
        allowed = int(np.floor(SPIKE_FLIP_FRACTION * self.n))
        return self.far_mismatch == 0 and self.spike_mismatch <= allowed and self.membrane_max_rel <= MEMBRANE_RTOL

    def __str__(self):
        return (f"n={self.n} spike_mismatch={self.spike_mismatch} far={self.far_mismatch} "
                f"membrane_max_rel={self.membrane_max_rel:.3e} over {self.membrane_compared}")


def compare(spikes_gpu: np.ndarray, h_gpu, spikes_ref: np.ndarray, h_ref: np.ndarray, v_th: float) -> ParityReport:
    """All arrays (T, ...) in the same element order.  h_gpu may be None (spikes only)."""
    s_g = spikes_gpu.astype(bool)
    s_r = spikes_ref.astype(bool)
    mism = s_g != s_r
    near = np.abs(h_ref - v_th) <= NEAR_THRESHOLD
    far = int(np.sum(mism & ~near))
    rel, cnt = 0.0, 0
    if h_gpu is not None:
        # compare step t only where spike histories agree on steps < t
        hist_ok = np.ones(s_g.shape[1:], bool)
        for t in range(s_g.shape[0]):
            sel = hist_ok
            if sel.any():
                err = np.abs(h_gpu[t][sel] - h_ref[t][sel]) / np.maximum(np.abs(h_ref[t][sel]), v_th)
                rel = max(rel, float(err.max()))
                cnt += int(sel.sum())
            hist_ok = hist_ok & ~mism[t]
    return ParityReport(int(s_g.size), int(mism.sum()), far, rel, cnt)


def nhwc_seq(x: torch.Tensor, T: int) -> np.ndarray:
    """(T*B, OH, OW, C) tensor -> numpy (T, B, C, OH, OW)."""
    a = x.detach().float().cpu().numpy()
    TB, OH, OW, C = a.shape
    return np.ascontiguousarray(a.reshape(T, TB // T, OH, OW, C).transpose(0, 1, 4, 2, 3))
