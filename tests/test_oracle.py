"""Pins the CPU oracle (oracle/) independently of the code it checks.

Each oracle function is checked against something the mathematics fixes — a closed form,
a brute-force evaluation or an invariant — chosen so that a plausible slip (a dropped
term, a wrong sign or index, a transposed operand) fails.  Runs on the CPU.
"""
import itertools
import math
import os

import numpy as np
import pytest
import torch

from oracle import packing as pk
from oracle import reference_path as ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "cfg0_golden.npz")


# ------------------------------------------------------------------------ neurons

def test_lif_no_spike_geometric_series():
    # below threshold forever: v_t = x (1 - 2^-(t+1)) for tau=2, constant x
    x = torch.full((6, 3), 0.9)
    s, h, _ = ref.multistep_lif(x, tau=2.0, v_threshold=1.0)
    assert s.sum() == 0
    for t in range(6):
        assert torch.allclose(h[t], torch.full((3,), 0.9 * (1 - 0.5 ** (t + 1))), rtol=0, atol=1e-7)


def test_lif_threshold_is_inclusive_and_hard_reset():
    # x=2, tau=2: v0 = 1.0 exactly == V_th -> spike (>=), reset to 0, repeats every step
    s, h, v = ref.multistep_lif(torch.full((4, 1), 2.0), tau=2.0, v_threshold=1.0, v_reset=0.0)
    assert s.flatten().tolist() == [1, 1, 1, 1]
    assert h.flatten().tolist() == [1.0, 1.0, 1.0, 1.0]
    assert v.item() == 0.0
    # x=1.9: 0.95 (no), 0.475+0.95=1.425 (spike), 0+0.95 (no), 1.425 (spike)
    s, h, _ = ref.multistep_lif(torch.full((4, 1), 1.9), tau=2.0, v_threshold=1.0)
    assert s.flatten().tolist() == [0, 1, 0, 1]
    assert np.allclose(h.flatten().numpy(), [0.95, 1.425, 0.95, 1.425], atol=1e-6)


def test_lif_general_tau_and_v_reset():
    tau, x, vr = 3.0, 2.1, 0.25
    s, h, _ = ref.multistep_lif(torch.full((3, 1), x), tau=tau, v_threshold=1.0, v_reset=vr)
    # hand trace in float64: v = v(1-1/tau) + x/tau
    v, hs, ss = 0.0, [], []
    for _ in range(3):
        v = v * (1 - 1 / tau) + x / tau
        hs.append(v)
        sp = v >= 1.0
        ss.append(float(sp))
        v = vr if sp else v
    assert s.flatten().tolist() == ss
    assert np.allclose(h.flatten().numpy(), hs, atol=1e-6)


def test_soft_reset_subtracts_threshold():
    # IF, x=1.5, soft reset: 1.5 (s) -> 0.5; 2.0 (s) -> 1.0; 2.5 (s) -> 1.5
    s, h, v = ref.multistep_if(torch.full((3, 1), 1.5), v_threshold=1.0, v_reset=None)
    assert s.flatten().tolist() == [1, 1, 1]
    assert h.flatten().tolist() == [1.5, 2.0, 2.5]
    assert v.item() == 1.5
    # LIF soft: tau=2, x=2.4: 1.2 (s)->0.2 ; 0.1+1.2=1.3 (s)->0.3 ; 0.15+1.2=1.35 (s)
    s, h, _ = ref.multistep_lif(torch.full((3, 1), 2.4), tau=2.0, v_threshold=1.0, v_reset=None)
    assert s.flatten().tolist() == [1, 1, 1]
    assert np.allclose(h.flatten().numpy(), [1.2, 1.3, 1.35], atol=1e-6)


def test_if_accumulates_without_leak():
    s, h, _ = ref.multistep_if(torch.full((5, 1), 0.3), v_threshold=1.0)
    assert np.allclose(h.flatten().numpy(), [0.3, 0.6, 0.9, 1.2, 0.3], atol=1e-6)
    assert s.flatten().tolist() == [0, 0, 0, 1, 0]


def test_initial_state_is_used():
    v0 = torch.tensor([0.8])
    s, h, _ = ref.multistep_lif(torch.full((1, 1), 1.2), tau=2.0, v0=v0)
    assert h.item() == pytest.approx(0.4 + 0.6) and s.item() == 1


# ------------------------------------------------------------------------ conv / BN

def brute_conv(x, w, stride, pad, dil):
    """float64 direct cross-correlation with zero padding."""
    N, C, H, W = x.shape
    K, _, KH, KW = w.shape
    OH = (H + 2 * pad - dil * (KH - 1) - 1) // stride + 1
    OW = (W + 2 * pad - dil * (KW - 1) - 1) // stride + 1
    out = np.zeros((N, K, OH, OW))
    for n, k, oh, ow in itertools.product(range(N), range(K), range(OH), range(OW)):
        acc = 0.0
        for c, r, s in itertools.product(range(C), range(KH), range(KW)):
            ih, iw = oh * stride - pad + r * dil, ow * stride - pad + s * dil
            if 0 <= ih < H and 0 <= iw < W:
                acc += float(x[n, c, ih, iw]) * float(w[k, c, r, s])
        out[n, k, oh, ow] = acc
    return out


@pytest.mark.parametrize("stride,pad,dil", [(1, 1, 1), (2, 1, 1), (1, 0, 1), (1, 2, 2), (2, 0, 1)])
def test_conv_bn_seq_matches_brute_force(stride, pad, dil):
    g = torch.Generator().manual_seed(3)
    T, B, C, H, W, K = 2, 2, 8, 5, 6, 4
    x = torch.bernoulli(torch.full((T, B, C, H, W), 0.4), generator=g)
    w = torch.randn((K, C, 3, 3), generator=g)
    bn = ref.BNParams(torch.rand(K, generator=g) + 0.5, torch.randn(K, generator=g), torch.randn(K, generator=g),
                      torch.rand(K, generator=g) + 0.5, 1e-5)
    y = ref.conv_bn_seq(x, w, bn, stride, pad, dil).numpy()
    conv = brute_conv(x.flatten(0, 1).numpy(), w.numpy(), stride, pad, dil)
    g64, b64, m64, v64 = (t.double().numpy()[None, :, None, None] for t in (bn.gamma, bn.beta, bn.mean, bn.var))
    expect = (conv - m64) / np.sqrt(v64 + 1e-5) * g64 + b64
    assert y.shape == (T, B, K) + expect.shape[2:]
    assert np.allclose(y.reshape(expect.shape), expect, rtol=1e-5, atol=1e-5)


def test_fold_batchnorm_closed_form():
    g = np.array([1.5, 0.5, 2.0]); b = np.array([0.1, -0.2, 0.0])
    m = np.array([0.3, -0.1, 2.0]); v = np.array([0.25, 4.0, 1.0 - 1e-5])
    scale, bias = ref.fold_batchnorm(g, b, m, v, 1e-5)
    exp_s = g / np.sqrt(v + 1e-5)
    assert np.allclose(scale, exp_s.astype(np.float32), rtol=0, atol=0)
    assert np.allclose(bias, (exp_s * (0 - m) + b).astype(np.float32), rtol=0, atol=0)
    assert scale[2] == np.float32(2.0) and bias[2] == np.float32(-4.0)
    x = np.linspace(-3, 3, 7)[:, None]
    assert np.allclose(x * scale + bias, (x - m) / np.sqrt(v + 1e-5) * g + b, atol=1e-5)
    _, bias_cb = ref.fold_batchnorm(g, b, m, v, 1e-5, conv_bias=np.array([1.0, 1.0, 1.0]))
    assert np.allclose(bias_cb, (exp_s * (1 - m) + b).astype(np.float32))


# ------------------------------------------------------------------------ 2:4 pruning

def test_prune_n_m_keeps_two_largest_per_group():
    g = torch.Generator().manual_seed(4)
    w = torch.randn((6, 16), generator=g)
    p = ref.prune_n_m(w)
    for r in range(6):
        for c0 in range(0, 16, 4):
            grp = w[r, c0:c0 + 4]
            keep = set(torch.argsort(grp.abs(), descending=True)[:2].tolist())
            for e in range(4):
                assert p[r, c0 + e].item() == (grp[e].item() if e in keep else 0.0)
    assert ref.verify_n_m(p)
    assert torch.equal(ref.prune_n_m(p), p)  # idempotent


def test_prune_n_m_pads_ragged_last_group():
    w = torch.tensor([[1.0, -5.0, 2.0, 0.5, 3.0, -4.0]])
    p = ref.prune_n_m(w)
    # group 1 = [3, -4, 0(pad), 0(pad)] keeps 3 and -4
    assert p.tolist() == [[0.0, -5.0, 2.0, 0.0, 3.0, -4.0]]


def test_prune_conv_groups_run_along_input_channels():
    g = torch.Generator().manual_seed(5)
    w = torch.randn((3, 8, 3, 3), generator=g)
    p = ref.prune_conv_2_4(w)
    for k, r, s in itertools.product(range(3), range(3), range(3)):
        for c0 in (0, 4):
            grp = w[k, c0:c0 + 4, r, s]
            keep = set(torch.argsort(grp.abs(), descending=True)[:2].tolist())
            got = p[k, c0:c0 + 4, r, s]
            assert [e for e in range(4) if got[e] != 0] == sorted(keep)
    assert ref.validate_2_4_pattern(p.numpy())
    assert not ref.validate_2_4_pattern(w.numpy())


def test_validate_and_verify_cases():
    ok = np.array([[1, 0, 2, 0, 0, 0, 3, 4.0]])
    assert ref.validate_2_4_pattern(ok) and ref.verify_n_m(torch.tensor(ok))
    three_zero = np.array([[1, 0, 0, 0]], np.float64)
    assert not ref.validate_2_4_pattern(three_zero) and not ref.verify_n_m(torch.tensor(three_zero))
    tiny = np.array([[1, 1e-12, 2, 0]])  # |w| < 1e-10 counts as zero for the engine check
    assert ref.validate_2_4_pattern(tiny) and not ref.verify_n_m(torch.tensor(tiny))
    assert not ref.validate_2_4_pattern(np.ones((2, 6)))  # cols % 4 != 0
    assert ref.verify_n_m(torch.ones(2, 3))  # no full group
    conv = np.zeros((1, 4, 1, 2)); conv[0, [0, 2], 0, 0] = 1; conv[0, [1, 3], 0, 1] = 1
    assert ref.validate_2_4_pattern(conv)


# ------------------------------------------------------------------------ packing

def test_pack_bits_known_answer():
    x = np.zeros((2, 64), np.float32)
    x[0, 0] = 1; x[0, 31] = 1; x[0, 33] = 1; x[1, 63] = 1
    words = pk.pack_bits(x)
    assert words.tolist() == [[0x80000001, 0x2], [0, 0x80000000]]
    assert np.array_equal(pk.unpack_bits(words, 64), x)


def test_seq_bits_roundtrip():
    g = np.random.default_rng(0)
    x = (g.random((2, 3, 64, 4, 5)) < 0.3).astype(np.float32)
    b = pk.seq_to_nhwc_bits(x)
    assert b.shape == (2 * 3 * 4 * 5, 2)
    assert np.array_equal(pk.nhwc_bits_to_seq(b, 2, 3, 64, 4, 5), x)
    # NHWC order: position ((t*B+b)*H+h)*W+w, channel c at bit c%32 of word c/32
    t, bb, c, h, w = 1, 2, 37, 3, 4
    pos = ((t * 3 + bb) * 4 + h) * 5 + w
    assert ((b[pos, c // 32] >> (c % 32)) & 1) == x[t, bb, c, h, w]


def test_compress_known_answer_slot():
    # one non-zero weight at (co=70, ci=133, kh=1, kw=2) of a 128->128 3x3 conv
    w = np.zeros((128, 192, 3, 3), np.float32)
    w[70, 133, 1, 2] = 0.625
    vals, meta, viol = pk.compress_2_4(w)
    v = vals.view(np.float16).astype(np.float32)
    k = (1 * 3 + 2) * 192 + 133           # reduction index (kh, kw, c_in)
    G, q = 70 // 64, k // 64              # group 1, chunk 23
    lane_group = (k % 64) // 16           # 4-group block inside the chunk -> lane // 16
    co_in_group = 70 - 64 * G             # 6 = 16*(r//4) + 4a + r%4 -> r//4 = 0, a = 1, r%4 = 2
    a, r = 1, 2
    lane = 16 * lane_group + r
    gi = (k % 16) // 4                    # 4-group inside the lane: 1, position 133 % 4 = 1
    nz = np.argwhere(v != 0)
    assert nz.tolist() == [[G, q, 0, a, lane, 2 * gi + 1]]  # kept positions {0? no: pad 0, 1} -> slot 1
    assert v[G, q, 0, a, lane, 2 * gi + 1] == 0.625
    assert ((meta[G, q, lane, a] >> (4 * gi)) & 0xF) == (0 | (1 << 2))  # positions (0, 1)
    assert viol.sum() == 0


def test_compress_roundtrip_and_planes():
    g = torch.Generator().manual_seed(6)
    w = ref.prune_conv_2_4(torch.randn((128, 64, 3, 3), generator=g) * 0.06).numpy()
    v1, m1, _ = pk.compress_2_4(w, planes=1)
    assert np.array_equal(pk.decompress_2_4(v1, m1, w.shape), w.astype(np.float16).astype(np.float32))
    v2, m2, _ = pk.compress_2_4(w, planes=2)
    back = pk.decompress_2_4(v2, m2, w.shape)
    assert np.array_equal(back == 0, w == 0)
    assert np.max(np.abs(back - w)) <= 2.0 ** -24 * 1.01 + np.max(np.abs(w)) * 2.0 ** -22


def test_compress_flags_violations():
    w = np.zeros((64, 64, 1, 1), np.float32)
    w[3, 0:3, 0, 0] = [1, 2, 3]      # three non-zeros in group (co=3, c 0..3)
    w[5, 4:6, 0, 0] = [1e-12, 7]     # 1e-12 counts as zero
    _, _, viol = pk.compress_2_4(w)
    assert viol.reshape(64, 16)[3, 0] == 1 and viol.sum() == 1


def test_dense_pack_roundtrip():
    g = np.random.default_rng(1)
    w = g.standard_normal((64, 96, 3, 3)).astype(np.float32)
    assert np.array_equal(pk.unpack_dense(pk.pack_dense(w, 1), w.shape), w.astype(np.float16).astype(np.float32))


# ------------------------------------------------------------------------ golden fixture

def test_golden_cfg0_reproduced_by_oracle():
    z = np.load(GOLDEN)
    c = ref.make_layer_case(0, T=4, B=1, C_in=64, C_out=64, H=32, W=32, k=3)
    assert np.array_equal(pk.seq_to_nhwc_bits(c.x_seq.numpy()), z["x_bits"])
    assert np.array_equal(c.w.numpy(), z["w"])
    assert ref.validate_2_4_pattern(z["w"])
    bn = ref.BNParams(*(torch.from_numpy(z[k]) for k in ("gamma", "beta", "mean", "var")), float(z["eps"]))
    r = ref.fused_layer(c.x_seq, c.w, bn, 1, 1, 1, "lif", 2.0, 1.0, 0.0)
    assert np.array_equal(pk.seq_to_nhwc_bits(r.spikes.numpy()), z["spikes_bits"])
    assert np.max(np.abs(r.h.numpy() - z["h"])) <= 1e-5
    # the config-0 statistics BASELINE.json fixes
    x = pk.nhwc_bits_to_seq(z["x_bits"], 4, 1, 64, 32, 32)
    assert abs(x.mean() - 0.15) < 0.005
    # kept weights are the 2 largest |w| of each 4-group of N(0, 2/576): their RMS is
    # sigma * sqrt(E[top-2-of-4 x^2]) = sigma * 1.3 within sampling error
    kept = z["w"][z["w"] != 0]
    assert kept.size == z["w"].size // 2
    assert math.isclose(float(np.sqrt(np.mean(kept ** 2))), (2 / 576) ** 0.5 * 1.3, rel_tol=0.15)


@pytest.mark.parametrize("H,W,k,stride,pad,dil", [(2, 2, 3, 1, 1, 1), (4, 4, 3, 2, 1, 1), (8, 8, 3, 2, 1, 1),
                                                 (4, 3, 1, 2, 0, 1), (1, 1, 3, 1, 1, 1), (5, 5, 3, 2, 2, 2)])
def test_flat_weight_is_the_conv(H, W, k, stride, pad, dil):
    """The flat small-output layout against torch's conv2d: NHWC-flattened images times the
    flat matrix equal the NHWC conv output."""
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(H * 10 + k)
    C_in, C_out, B = 8, 12, 3
    x = torch.randn(B, C_in, H, W, generator=g, dtype=torch.float64)
    w = torch.randn(C_out, C_in, k, k, generator=g, dtype=torch.float64)
    y = F.conv2d(x, w, None, stride, pad, dil)  # (B, C_out, OH, OW)
    flat = torch.from_numpy(pk.flat_weight(w.numpy(), H, W, stride, pad, dil))[:, :, 0, 0]
    got = x.permute(0, 2, 3, 1).reshape(B, -1) @ flat.T
    assert torch.allclose(got, y.permute(0, 2, 3, 1).reshape(B, -1), atol=1e-12)


def test_ms_neuron_closed_forms():
    """MSNeuron (decay 1/4, threshold 1/2) on constant inputs with exact binary fractions:
    x = 3/8 approaches 1/2 from below and never fires; x = 1/2 fires at every step (each
    spike zeroes the carried membrane); x = 7/16 charges to 35/64 >= 1/2 and fires every
    other step; a negative input never fires and the membrane follows x * sum(decay^k)."""
    T = 6
    x = torch.tensor([0.375, 0.5, 0.4375, -0.25]).view(1, 4).repeat(T, 1)
    s, h, _ = ref.ms_neuron(x, 0.25, 0.5)
    assert s[:, 0].sum() == 0
    assert torch.equal(s[:, 1], torch.ones(T))
    assert torch.equal(s[:, 2], torch.tensor([0.0, 1, 0, 1, 0, 1]))
    assert h[1, 2] == 0.546875 and h[2, 2] == 0.4375
    geo = torch.tensor([sum(0.25 ** k for k in range(t + 1)) for t in range(T)])
    assert torch.allclose(h[:, 0], 0.375 * geo) and torch.allclose(h[:, 3], -0.25 * geo)
    assert s[:, 3].sum() == 0
    # initial membrane: charged once by decay, then the input
    s0, h0, _ = ref.ms_neuron(x[:, :1], 0.25, 0.5, v0=torch.tensor([1.0]))
    assert h0[0, 0] == 0.625 and s0[0, 0] == 1 and h0[1, 0] == 0.375


def test_shortcut_layer_composition():
    """The membrane-shortcut layer is conv+BN, plus the residual, then the neuron."""
    case = ref.make_layer_case(3, T=3, B=1, C_in=8, C_out=8, H=5, W=5, k=3)
    res = torch.randn(3, 1, 8, 5, 5, generator=torch.Generator().manual_seed(1))
    r = ref.shortcut_layer(case.x_seq, case.w, case.bn, res, 1, 1, "ms", 0.25, 0.5)
    y = ref.conv_bn_seq(case.x_seq, case.w, case.bn, 1, 1) + res
    assert torch.equal(r.x, y)
    assert torch.equal(r.spikes, ref.ms_neuron(y, 0.25, 0.5)[0])
