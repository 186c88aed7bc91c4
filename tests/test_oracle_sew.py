"""Pins of the SEW-ResNet-18 restatement (oracle/sew_resnet.py) beyond its pinned parts:
the stem against a numpy direct convolution, max/avg pooling, the block wiring (ADD of the
right tensors), the head, and the bit-plane format of integer activations."""
import numpy as np
import torch

from oracle import packing as pk
from oracle import reference_path as ref
from oracle import sew_resnet as sr


def _np_conv(x, w, stride, pad):
    N, C, H, W = x.shape
    F, _, K, _ = w.shape
    xp = np.pad(x, ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    OH, OW = (H + 2 * pad - K) // stride + 1, (W + 2 * pad - K) // stride + 1
    out = np.zeros((N, F, OH, OW))
    for kh in range(K):
        for kw in range(K):
            patch = xp[:, :, kh:kh + stride * OH:stride, kw:kw + stride * OW:stride]
            out += np.einsum("nchw,fc->nfhw", patch, w[:, :, kh, kw])
    return out


def _run(seed=3, B=2):
    p = sr.make_params(seed, bn_random=True, fp16_weights=True)
    x = sr.make_images(seed + 1, B)
    rec = {}
    y = sr.forward(p, x, record=rec)
    return p, x, rec, y


def test_params_are_2_4_except_stem_and_use_reference_names():
    p = sr.make_params(0)
    names = [n for n, *_ in sr.conv_names()]
    assert names[0] == "conv1" and "layer2.0.downsample.0.module.0" in names and len(names) == 20
    for n in names[1:]:
        assert ref.verify_n_m(ref.conv_weight_2d(p[n + ".weight"]))
    assert bool((p["conv1.weight"] != 0).all())  # the stem stays dense (C_in = 3)
    assert p["fc.weight"].shape == (100, 512)


def test_stem_matches_numpy_conv_bn_and_repeated_neuron():
    p, x, rec, _ = _run()
    conv = _np_conv(x.double().numpy(), p["conv1.weight"].double().numpy(), 2, 3)
    sc, bi = ref.fold_batchnorm(p["bn1.weight"], p["bn1.bias"], p["bn1.running_mean"], p["bn1.running_var"])
    bn = conv * sc[None, :, None, None] + bi[None, :, None, None]
    s, _, _ = ref.multistep_lif(torch.from_numpy(np.repeat(bn[None], 4, 0)).float())
    near = np.abs(np.repeat(bn[None], 4, 0) / 2 - 1.0) < 1e-4
    assert np.all((s.numpy() == rec["stem"].numpy()) | near)
    assert 0.01 < float(rec["stem"].mean()) < 0.5


def test_maxpool_is_window_or_of_spikes():
    _, _, rec, _ = _run()
    s = rec["stem"].numpy()
    T, B, C, H, W = s.shape
    sp = np.pad(s, ((0, 0), (0, 0), (0, 0), (1, 1), (1, 1)))
    exp = np.zeros((T, B, C, H // 2, W // 2))
    for kh in range(3):
        for kw in range(3):
            exp = np.maximum(exp, sp[:, :, :, kh:kh + H:2, kw:kw + W:2])
    assert np.array_equal(exp, rec["maxpool"].numpy())


def test_block_wiring_adds_spikes_to_identity():
    _, _, rec, _ = _run()
    prev = "maxpool"
    for si in range(4):
        for bi in range(2):
            pre = f"layer{si + 1}.{bi}"
            ident = rec[pre + ".downsample"] if (pre + ".downsample") in rec else rec[prev]
            assert torch.equal(rec[pre], rec[pre + ".sn2"] + ident)
            prev = pre
    assert "layer1.0.downsample" not in rec and "layer2.0.downsample" in rec
    assert float(rec["layer1.1"].max()) <= 3 and float(rec["layer4.1"].max()) <= 3


def test_head_is_mean_over_space_and_time_then_linear():
    p, _, rec, y = _run()
    a = rec["layer4.1"].double().numpy()
    feat = a.mean(axis=(3, 4)).mean(axis=0)
    exp = feat @ p["fc.weight"].double().numpy().T + p["fc.bias"].double().numpy()
    assert np.allclose(y.double().numpy(), exp, atol=1e-5)


def test_bit_planes_roundtrip_and_layout():
    rng = np.random.default_rng(0)
    x = rng.integers(0, 4, size=(2, 3, 64, 2, 3))
    w = pk.seq_to_planes(x, 2)
    assert w.shape == (2 * 3 * 2 * 3, 4)
    assert np.array_equal(pk.planes_to_seq(w, 2, 2, 3, 64, 2, 3), x.astype(np.float32))
    # channel c of plane 1 is bit 1 of x[..., c]: word 2 bit 0 is channel 0 of plane 1
    pos0 = x[0, 0, :, 0, 0]
    assert ((w[0, 2] >> 0) & 1) == (pos0[0] >> 1) & 1
