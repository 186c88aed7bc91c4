"""Parity helpers shared by the GPU tests, smoke() and bench.py.

Acceptance rule (output spikes bit-exact except for a fraction
<= 1e-4 of neurons whose reference membrane lies within 1e-3 of threshold), applied per layer
call:
  * at most floor(1e-4 * n_neurons) distinct neurons may have any spike mismatch (a neuron is
    one output element over its T steps);
  * a neuron's first mismatch (its spike history agreed with the reference up to the
    previous step) must have a reference membrane within 1e-3 of V_th at that step;
  * its later mismatches are consequences of that flip -- one side reset, the other did
    not, so the two membrane trajectories differ from then on -- and are allowed at any
    membrane distance: they belong to a neuron already counted in the budget;
  * charged membranes within 1e-3 * max(|v_ref|, V_th), compared wherever the spike
    history of the neuron agrees with the reference up to the previous step.
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
    spike_mismatch: int    # all mismatching neuron-steps
    far_mismatch: int      # first flips of a neuron whose reference membrane is not near threshold
    membrane_max_rel: float
    membrane_compared: int
    flips: int = 0         # first mismatches = distinct neurons whose spike history diverged
    neurons: int = 0       # neurons compared (n / T)

    @property
    def allowed(self) -> int:
        return int(np.floor(SPIKE_FLIP_FRACTION * self.neurons))

    @property
    def ok(self) -> bool:
        return self.far_mismatch == 0 and self.flips <= self.allowed and self.membrane_max_rel <= MEMBRANE_RTOL

    def __str__(self):
        return (f"n={self.n} neurons={self.neurons} mismatching neurons={self.flips} (allowed {self.allowed}; "
                f"{self.spike_mismatch} neuron-steps, {self.spike_mismatch - self.flips} after a flip) "
                f"far={self.far_mismatch} membrane_max_rel={self.membrane_max_rel:.3e} over {self.membrane_compared}")


def compare(spikes_gpu: np.ndarray, h_gpu, spikes_ref: np.ndarray, h_ref: np.ndarray, v_th: float) -> ParityReport:
    """All arrays (T, ...) in the same element order.  h_gpu may be None (spikes only)."""
    s_g = spikes_gpu.astype(bool)
    s_r = spikes_ref.astype(bool)
    mism = s_g != s_r
    rel, cnt, far, flips = 0.0, 0, 0, 0
    hist_ok = np.ones(s_g.shape[1:], bool)  # spike histories agree on steps < t
    for t in range(s_g.shape[0]):
        first = mism[t] & hist_ok
        if first.any():
            flips += int(first.sum())
            far += int(np.sum(np.abs(h_ref[t][first] - v_th) > NEAR_THRESHOLD))
        if h_gpu is not None and hist_ok.any():
            sel = hist_ok
            err = np.abs(h_gpu[t][sel] - h_ref[t][sel]) / np.maximum(np.abs(h_ref[t][sel]), v_th)
            rel = max(rel, float(err.max()))
            cnt += int(sel.sum())
        hist_ok = hist_ok & ~mism[t]
    return ParityReport(int(s_g.size), int(mism.sum()), far, rel, cnt, flips, int(s_g[0].size))


def compare_final(v_gpu: np.ndarray, v_ref: np.ndarray, spikes_gpu: np.ndarray, spikes_ref: np.ndarray,
                  v_th: float):
    """Final membranes (after the last reset), compared where the neuron's whole spike history
    agrees with the reference (an allowed near-threshold flip legitimately changes the
    trajectory).  spikes_* (T, ...) and v_* (...) in the same element order.  Returns
    (max relative error, neurons compared)."""
    same = np.all(spikes_gpu.astype(bool) == spikes_ref.astype(bool), axis=0)
    if not same.any():
        return 0.0, 0
    err = np.abs(v_gpu[same] - v_ref[same]) / np.maximum(np.abs(v_ref[same]), v_th)
    return float(err.max()), int(same.sum())


def nhwc_seq(x: torch.Tensor, T: int) -> np.ndarray:
    """(T*B, OH, OW, C) tensor -> numpy (T, B, C, OH, OW)."""
    a = x.detach().float().cpu().numpy()
    TB, OH, OW, C = a.shape
    return np.ascontiguousarray(a.reshape(T, TB // T, OH, OW, C).transpose(0, 1, 4, 2, 3))
