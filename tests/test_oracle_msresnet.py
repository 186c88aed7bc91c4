"""Pins of the MS-ResNet restatement (oracle/ms_resnet.py) beyond its pinned parts: the TDBN
container against a literal BatchNorm3d on the (B, C, T, H, W) permutation, the stem's
T-invariance, the block wiring (membrane shortcut: identity or 1x1 conv of the real-valued
input, added after conv_bn2) on hand-built special cases, the head against numpy, and the
parameter names / 2:4 structure."""
import numpy as np
import torch

from oracle import ms_resnet as ms
from oracle import reference_path as ref


def _tiny_params(seed=0, depth=18):
    return ms.make_params(seed, depth, num_classes=10, init="lively", fp16_weights=True)


def test_params_use_reference_names_and_are_2_4():
    p = ms.make_params(0, 34, init="reference")
    names = ms.block_names(34)
    assert len(names) == 16 and names[0][0] == "conv2_x.0" and names[-1][0] == "conv5_x.2"
    assert [n for n, *_, sc in names if sc] == ["conv2_x.0", "conv3_x.0", "conv4_x.0", "conv5_x.0"]
    for pre, *_, has_sc in names:
        for c in ("conv_bn1", "conv_bn2") + (("shortcut",) if has_sc else ()):
            w = p[f"{pre}.{c}.module.0.weight"]
            assert ref.verify_n_m(ref.conv_weight_2d(w))
    assert bool((p["conv1.module.0.weight"] != 0).all())  # the stem stays dense (C_in = 3)
    # bn_init_thresh: 0.5 on conv1 / conv_bn1 / shortcut, default 1 on conv_bn2 (models/msresnet.py:75-76)
    assert float(p["conv1.module.1.weight"][0]) == 0.5
    assert float(p["conv2_x.0.conv_bn1.module.1.weight"][0]) == 0.5
    assert float(p["conv2_x.0.conv_bn2.module.1.weight"][0]) == 1.0
    assert float(p["conv2_x.0.shortcut.module.1.weight"][0]) == 0.5
    assert p["fc.weight"].shape == (1000, 512)


def test_tdbn_equals_batchnorm3d_on_the_permuted_tensor():
    g = torch.Generator().manual_seed(1)
    T, B, C, F, H = 3, 2, 8, 16, 7
    x = torch.randn(T, B, C, H, H, generator=g)
    w = torch.randn(F, C, 3, 3, generator=g) * 0.2
    bn3 = torch.nn.BatchNorm3d(F).eval()
    with torch.no_grad():
        bn3.weight.copy_(torch.rand(F, generator=g) + 0.5)
        bn3.bias.copy_(torch.randn(F, generator=g) * 0.1)
        bn3.running_mean.copy_(torch.randn(F, generator=g) * 0.1)
        bn3.running_var.copy_(torch.rand(F, generator=g) + 0.5)
        conv = torch.nn.functional.conv2d(x.flatten(0, 1), w, None, 2, 1)
        lit = bn3(conv.view(T, B, *conv.shape[1:]).permute(1, 2, 0, 3, 4)).permute(2, 0, 1, 3, 4)
    bn = ref.BNParams(bn3.weight.detach(), bn3.bias.detach(), bn3.running_mean, bn3.running_var, bn3.eps)
    out = ms.tdbn(x, w, bn, 2, 1)
    assert out.shape == lit.shape
    assert torch.allclose(out, lit, rtol=1e-6, atol=1e-6)


def test_stem_is_the_same_for_every_timestep():
    p = _tiny_params()
    x = torch.randn(2, 3, 32, 32, generator=torch.Generator().manual_seed(2))
    y = ms.stem(p, x, 4)
    assert y.shape == (4, 2, 64, 16, 16)
    for t in range(1, 4):
        assert torch.equal(y[t], y[0])


def _block_with(p, pre, **over):
    q = dict(p)
    q.update(over)
    return q


def test_block_identity_shortcut_adds_the_real_input():
    """conv_bn2 with zero weights leaves BN2's bias: out = bias2 + x exactly (identity shortcut)."""
    p = _tiny_params()
    pre = "conv2_x.1"  # stride 1, 64 -> 64: identity shortcut
    C = 64
    bias2 = torch.randn(C, generator=torch.Generator().manual_seed(5))
    q = _block_with(p, pre, **{pre + ".conv_bn2.module.0.weight": torch.zeros(C, C, 3, 3),
                               pre + ".conv_bn2.module.1.weight": torch.ones(C),
                               pre + ".conv_bn2.module.1.bias": bias2,
                               pre + ".conv_bn2.module.1.running_mean": torch.zeros(C),
                               pre + ".conv_bn2.module.1.running_var": torch.full((C,), 1.0 - 1e-5)})
    x = torch.randn(2, 2, C, 5, 5, generator=torch.Generator().manual_seed(6))
    out = ms.block_forward(q, pre, x, 1, False, "ms", 0.25, 0.5)
    assert torch.allclose(out, x + bias2[None, None, :, None, None], rtol=0, atol=1e-6)


def test_block_conv_shortcut_reads_the_real_input_not_spikes():
    """With conv_bn2 zeroed as above, a stride-2 block returns bias2 + TDBN(1x1/2 conv of x):
    the shortcut convolves the real-valued x (a spike input would give a different value)."""
    p = _tiny_params()
    pre = "conv3_x.0"  # stride 2, 64 -> 128, shortcut conv
    Ci, Co = 64, 128
    q = _block_with(p, pre, **{pre + ".conv_bn2.module.0.weight": torch.zeros(Co, Co, 3, 3),
                               pre + ".conv_bn2.module.1.weight": torch.ones(Co),
                               pre + ".conv_bn2.module.1.bias": torch.zeros(Co),
                               pre + ".conv_bn2.module.1.running_mean": torch.zeros(Co),
                               pre + ".conv_bn2.module.1.running_var": torch.full((Co,), 1.0 - 1e-5)})
    x = torch.randn(2, 2, Ci, 6, 6, generator=torch.Generator().manual_seed(7))
    out = ms.block_forward(q, pre, x, 2, True, "lif", 2.0, 1.0)
    w = p[pre + ".shortcut.module.0.weight"].double().numpy()[:, :, 0, 0]
    sc, bi = ref.fold_batchnorm(p[pre + ".shortcut.module.1.weight"], p[pre + ".shortcut.module.1.bias"],
                                p[pre + ".shortcut.module.1.running_mean"], p[pre + ".shortcut.module.1.running_var"])
    xs = x.double().numpy()[:, :, :, ::2, ::2]
    exp = np.einsum("tbchw,fc->tbfhw", xs, w) * sc[None, None, :, None, None] + bi[None, None, :, None, None]
    assert np.allclose(out.double().numpy(), exp, atol=1e-4)


def test_block_spike_path_uses_sn1_then_conv_bn1_then_sn2():
    """With the shortcut contribution removed (x = 0 on the identity path is not possible, so
    compare out - x): out - x == TDBN2(sn2(TDBN1(sn1(x))))."""
    p = _tiny_params()
    pre = "conv2_x.1"
    x = torch.randn(3, 2, 64, 6, 6, generator=torch.Generator().manual_seed(8)) * 0.8
    out = ms.block_forward(p, pre, x, 1, False, "ms", 0.25, 0.5)
    s1 = ref.ms_neuron(x, 0.25, 0.5)[0]
    y1 = ref.conv_bn_seq(s1, p[pre + ".conv_bn1.module.0.weight"], ms.bn_of(p, pre + ".conv_bn1.module.1"), 1, 1)
    s2 = ref.ms_neuron(y1, 0.25, 0.5)[0]
    y2 = ref.conv_bn_seq(s2, p[pre + ".conv_bn2.module.0.weight"], ms.bn_of(p, pre + ".conv_bn2.module.1"), 1, 1)
    assert torch.equal(out, y2 + x)
    assert 0.02 < float(s1.mean()) < 0.9 and 0.02 < float(s2.mean()) < 0.9


def test_head_is_mean_over_time_then_space_then_linear():
    p = _tiny_params()
    g = torch.Generator().manual_seed(9)
    s = (torch.rand(4, 2, 512, 3, 3, generator=g) < 0.3).float()
    y = ms.head(p, s)
    feat = s.double().numpy().mean(axis=0).mean(axis=(2, 3))
    exp = feat @ p["fc.weight"].double().numpy().T + p["fc.bias"].double().numpy()
    assert np.allclose(y.double().numpy(), exp, atol=1e-5)


def test_forward_shapes_and_activity():
    p = _tiny_params(depth=18)
    x = torch.randn(2, 3, 64, 64, generator=torch.Generator().manual_seed(10))
    logits, xs = ms.forward(p, x, T=4, depth=18, kind="lif", tau=2.0, v_threshold=1.0, keep=True)
    assert logits.shape == (2, 10) and len(xs) == 9
    assert xs[0].shape == (4, 2, 64, 32, 32) and xs[-1].shape == (4, 2, 512, 2, 2)
    rates = [float(ms.neuron(v, "lif", 2.0, 1.0).mean()) for v in xs]
    assert all(0.01 < r < 0.9 for r in rates), rates
