"""CPU restatement of MS-ResNet-18/34 inference — TEST INFRASTRUCTURE ONLY.

Follows models/msresnet.py of the reference:
  * TDBNContainer (:58-80): Conv2d on the flattened (T*B) batch, then BatchNorm3d on the
    (B, C, T, H, W) permutation — in eval mode a per-channel affine, i.e. the same values
    as conv_bn_seq's BatchNorm2d on (T*B, C, H, W) (pinned in tests/test_oracle_msresnet.py);
  * MSNeuron (:28-56): mem = mem * decay * (1 - spike) + x, spike = (mem - thresh) >= 0,
    decay 0.25, thresh 0.5 (:21-22);
  * BasicBlock18 (:87-112): out = conv_bn2(sn2(conv_bn1(sn1(x)))) + shortcut(x), the
    shortcut a 1x1/stride TDBN conv on the real-valued x when the stride or width changes,
    else x itself (the membrane shortcut: x is never a spike tensor here);
  * MSResNet18 (:119-161): the image repeated over T (:146-150), conv1 = TDBN(7x7/2, pad 3)
    with no neuron and no max-pool, four stages whose first block has stride 2
    (_make_layer(..., 2) for every stage, :130-133), sn_out, mean over T, adaptive average
    pool, Linear; ms_resnet34 = [3, 4, 6, 3] blocks (:318-319), ms_resnet18 = [2, 2, 2, 2].
The neuron is selectable: 'ms' (the reference's MSNeuron) or 'lif' (BASELINE config 3's
LIF tau 2, V_th 1, models/neurons.py:121-146 with hard reset to 0).

Parameters use the reference's state_dict key names (conv1.module.0/1,
conv{2..5}_x.{i}.conv_bn{1,2}.module.{0,1}, ...shortcut.module.{0,1}, fc).

Pinning: conv_bn_seq (float64 brute-force convolution), ms_neuron / multistep_lif (closed
forms) are pinned in tests/test_oracle.py; tests/test_oracle_msresnet.py checks the TDBN
equivalence above against a literal BatchNorm3d on the permuted tensor, the block wiring
against a hand-built composition, the stem's T-invariance and the head against numpy.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .reference_path import BNParams, conv_bn_seq, ms_neuron, multistep_lif, prune_conv_2_4

DEPTHS = {18: (2, 2, 2, 2), 34: (3, 4, 6, 3)}
WIDTHS = (64, 128, 256, 512)
MS_DECAY, MS_THRESH = 0.25, 0.5  # models/msresnet.py:21-22


def block_names(depth: int = 34):
    """(prefix, C_in, C_out, stride, has_shortcut) of every BasicBlock18 in forward order."""
    out, cin = [], 64
    for si, (planes, n) in enumerate(zip(WIDTHS, DEPTHS[depth])):
        for bi in range(n):
            s = 2 if bi == 0 else 1
            out.append((f"conv{si + 2}_x.{bi}", cin, planes, s, s != 1 or cin != planes))
            cin = planes
    return out


def make_params(seed: int = 0, depth: int = 34, num_classes: int = 1000, in_channels: int = 3, prune: bool = True,
                init: str = "lively", fp16_weights: bool = False) -> dict:
    """Random ms_resnet{18,34} parameters keyed by the reference's state_dict names.

    init='reference': PyTorch's defaults as the reference model gets them (Conv2d
    kaiming_uniform(a=sqrt(5)) = U(+-1/sqrt(fan_in)); BatchNorm3d weight 0.5 where
    bn_init_thresh (conv1, conv_bn1, shortcut; models/msresnet.py:75-76) else 1, bias 0,
    running mean 0 / var 1; Linear U(+-1/sqrt(fan_in))).
    init='lively': conv weights N(0, 2/fan_in), BN gamma~U(0.5,1.5), beta~N(0,0.1),
    mean~N(0,0.1), var~U(0.5,1.5) (BASELINE config 0's draws), so that every layer spikes
    (tests need activity to mean anything).
    prune: 2:4 magnitude mask along C_in on every conv but the stem."""
    g = torch.Generator().manual_seed(seed)
    p = {}

    def conv(name, cin, cout, k, do_prune):
        fan_in = cin * k * k
        if init == "reference":
            b = 1.0 / math.sqrt(fan_in)
            w = (torch.rand((cout, cin, k, k), generator=g) * 2 - 1) * b
        else:
            w = torch.randn((cout, cin, k, k), generator=g) * math.sqrt(2.0 / fan_in)
        if do_prune:
            w = prune_conv_2_4(w)
            if fp16_weights:
                w = w.half().float()
        p[name + ".weight"] = w

    def bn(name, c, thresh_init):
        if init == "reference":
            p[name + ".weight"] = torch.full((c,), MS_THRESH if thresh_init else 1.0)
            p[name + ".bias"] = torch.zeros(c)
            p[name + ".running_mean"], p[name + ".running_var"] = torch.zeros(c), torch.ones(c)
        else:
            p[name + ".weight"] = torch.rand(c, generator=g) + 0.5
            p[name + ".bias"] = torch.randn(c, generator=g) * 0.1
            p[name + ".running_mean"] = torch.randn(c, generator=g) * 0.1
            p[name + ".running_var"] = torch.rand(c, generator=g) + 0.5

    conv("conv1.module.0", in_channels, 64, 7, False)
    bn("conv1.module.1", 64, True)
    for pre, cin, cout, s, has_sc in block_names(depth):
        conv(pre + ".conv_bn1.module.0", cin, cout, 3, prune)
        bn(pre + ".conv_bn1.module.1", cout, True)
        conv(pre + ".conv_bn2.module.0", cout, cout, 3, prune)
        bn(pre + ".conv_bn2.module.1", cout, False)
        if has_sc:
            conv(pre + ".shortcut.module.0", cin, cout, 1, prune)
            bn(pre + ".shortcut.module.1", cout, True)
    bound = 1.0 / math.sqrt(512)
    p["fc.weight"] = (torch.rand((num_classes, 512), generator=g) * 2 - 1) * bound
    p["fc.bias"] = (torch.rand(num_classes, generator=g) * 2 - 1) * bound
    return p


def bn_of(p: dict, name: str) -> BNParams:
    return BNParams(p[name + ".weight"], p[name + ".bias"], p[name + ".running_mean"], p[name + ".running_var"], 1e-5)


def tdbn(x_seq: torch.Tensor, w: torch.Tensor, bn: BNParams, stride: int, padding: int) -> torch.Tensor:
    """TDBNContainer.forward (models/msresnet.py:69-80) in eval mode: (T, B, C, H, W) ->
    (T, B, C', H', W'); BatchNorm3d over the (B, C, T, H, W) view is per-channel, so this is
    conv_bn_seq (the equivalence is pinned against a literal BatchNorm3d in the tests)."""
    return conv_bn_seq(x_seq, w, bn, stride, padding)


def neuron(x_seq: torch.Tensor, kind: str, tau: float, v_threshold: float) -> torch.Tensor:
    """The block neuron: 'ms' = MSNeuron(decay=tau, thresh=v_threshold) (:28-56), 'lif' =
    MultiStepLIFNeuron(tau, v_threshold, hard reset to 0) (models/neurons.py:187-211)."""
    if kind == "ms":
        return ms_neuron(x_seq, tau, v_threshold)[0]
    return multistep_lif(x_seq, tau, v_threshold, 0.0)[0]


def block_forward(p: dict, pre: str, x: torch.Tensor, stride: int, has_sc: bool, kind: str, tau: float,
                  v_threshold: float) -> torch.Tensor:
    """BasicBlock18.forward (models/msresnet.py:107-112) on the real-valued block input x."""
    out = tdbn(neuron(x, kind, tau, v_threshold), p[pre + ".conv_bn1.module.0.weight"],
               bn_of(p, pre + ".conv_bn1.module.1"), stride, 1)
    out = tdbn(neuron(out, kind, tau, v_threshold), p[pre + ".conv_bn2.module.0.weight"],
               bn_of(p, pre + ".conv_bn2.module.1"), 1, 1)
    sc = tdbn(x, p[pre + ".shortcut.module.0.weight"], bn_of(p, pre + ".shortcut.module.1"), stride, 0) \
        if has_sc else x
    return out + sc


def stem(p: dict, x_img: torch.Tensor, T: int) -> torch.Tensor:
    """Input repeated over T (:146-150), then conv1 = TDBN(7x7/2, pad 3) (:125-128)."""
    seq = x_img.unsqueeze(0).repeat(T, 1, 1, 1, 1)
    return tdbn(seq, p["conv1.module.0.weight"], bn_of(p, "conv1.module.1"), 2, 3)


def head(p: dict, spikes: torch.Tensor) -> torch.Tensor:
    """sn_out's spikes -> mean over T, adaptive average pool, flatten, Linear (:155-160)."""
    out = spikes.mean(dim=0)
    out = F.adaptive_avg_pool2d(out, 1).flatten(1)
    return F.linear(out, p["fc.weight"], p["fc.bias"])


def forward(p: dict, x_img: torch.Tensor, T: int = 4, depth: int = 34, kind: str = "ms", tau: float = MS_DECAY,
            v_threshold: float = MS_THRESH, keep: bool = False):
    """MSResNet18.forward (models/msresnet.py:144-161) for images (B, C, H, W).
    Returns logits, or (logits, [block inputs x_0 .. x_n]) with keep=True (x_n = the last
    block's output, whose neuron is sn_out)."""
    with torch.no_grad():
        x = stem(p, x_img.float(), T)
        xs = [x]
        for pre, _, _, s, has_sc in block_names(depth):
            x = block_forward(p, pre, x, s, has_sc, kind, tau, v_threshold)
            xs.append(x)
        logits = head(p, neuron(x, kind, tau, v_threshold))
    return (logits, xs) if keep else logits
