"""The acceptance rule of tests/parity.py on planted CPU cases: the LIF trajectories come from
the oracle (models/neurons.py:121-146) on inputs that differ in chosen places."""
import numpy as np
import torch

from oracle import reference_path as ref
from tests.parity import compare, compare_final


def _lif(x):
    s, h, v = ref.multistep_lif(torch.from_numpy(x), 2.0, 1.0, 0.0)
    return s.numpy(), h.numpy(), v.numpy()


def _base(n=20000, seed=0):
    x = np.random.default_rng(seed).uniform(0.0, 1.2, size=(4, n)).astype(np.float32)
    return x


def test_identical_runs_pass():
    x = _base()
    s, h, _ = _lif(x)
    rep = compare(s, h, s, h, 1.0)
    assert rep.ok and rep.spike_mismatch == 0 and rep.flips == 0


def test_near_threshold_flip_and_its_consequences_pass():
    """Reference h at t=1 sits 4e-4 below V_th; the other side sits just above it and fires,
    resets, and so misses the reference's (far-from-threshold) spike at t=2."""
    x = _base(seed=1)
    x[:, 0] = [1.0, 1.4992, 1.8, 0.0]  # h0 = 0.5, h1 = 0.25 + 0.7496 = 0.9996: 4e-4 below V_th
    s_r, h_r, _ = _lif(x)
    assert s_r[1, 0] == 0 and abs(h_r[1, 0] - 1.0) < 1e-3 and s_r[2, 0] == 1  # h2 = 0.4998 + 0.9 >= 1
    xg = x.copy()
    xg[1, 0] = 1.5004  # h1 = 1.0002: fires
    s_g, h_g, _ = _lif(xg)
    assert s_g[1, 0] == 1 and s_g[2, 0] == 0  # reset to 0, then h2 = 0.9 < 1
    rep = compare(s_g, h_g, s_r, h_r, 1.0)
    assert rep.flips == 1 and rep.spike_mismatch == 2 and rep.far_mismatch == 0, str(rep)
    assert rep.ok, str(rep)


def test_far_first_flip_fails():
    x = _base(seed=2)
    s_r, h_r, _ = _lif(x)
    i = int(np.argmin(np.abs(h_r[0] - 0.5)))  # a neuron at h = 0.5 at t = 0
    s_g = s_r.copy()
    s_g[0, i] = 1.0
    rep = compare(s_g, None, s_r, h_r, 1.0)
    assert rep.far_mismatch == 1 and not rep.ok


def test_flip_budget():
    """Near-threshold flips are allowed in at most 1e-4 of the neurons (not of the neuron-steps:
    T = 4 steps per neuron would allow four times as many)."""
    n = 20000  # 20,000 neurons (80,000 neuron-steps): 2 mismatching neurons allowed
    x = np.full((4, n), 0.3, np.float32)
    x[0, :] = 1.9995  # h0 = 0.99975 at every neuron: near threshold, no reference spike
    s_r, h_r, _ = _lif(x)
    for k, ok in ((2, True), (3, False), (8, False)):
        s_g = s_r.copy()
        s_g[0, :k] = 1.0  # first flips only, near threshold; later steps kept equal
        rep = compare(s_g, None, s_r, h_r, 1.0)
        assert rep.flips == k and rep.far_mismatch == 0 and rep.ok == ok, (k, str(rep))


def test_budget_counts_neurons_not_steps():
    """Two neurons that each mismatch at several steps after a near-threshold first flip use two
    units of the budget, not one per mismatching step."""
    n = 20000  # 2 neurons allowed
    x = np.full((4, n), 0.3, np.float32)
    x[0, :] = 1.9995
    s_r, h_r, _ = _lif(x)
    s_g = s_r.copy()
    s_g[:, :2] = 1.0  # neurons 0 and 1 differ at all four steps
    rep = compare(s_g, None, s_r, h_r, 1.0)
    assert rep.spike_mismatch == 8 and rep.flips == 2 and rep.ok, str(rep)
    s_g[:, 2] = 1.0  # a third neuron: over budget
    assert not compare(s_g, None, s_r, h_r, 1.0).ok


def test_membrane_tolerance():
    x = _base(seed=3)
    s, h, v = _lif(x)
    hg = h.copy()
    hg[2, 5] = h[2, 5] + 0.9e-3 * max(abs(h[2, 5]), 1.0)
    assert compare(s, hg, s, h, 1.0).ok
    hg[2, 5] = h[2, 5] + 1.1e-3 * max(abs(h[2, 5]), 1.0)
    assert not compare(s, hg, s, h, 1.0).ok
    vg = v.copy()
    vg[7] += 2e-3
    rel, n = compare_final(vg, v, s, s, 1.0)
    assert n == v.size and rel > 1e-3
