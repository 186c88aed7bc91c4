"""CPU restatement of SEW-ResNet-18 inference — TEST INFRASTRUCTURE ONLY.

Follows models/sewresnet.py of the reference: BasicBlock (:27-66) with the SEW 'ADD'
connection (:58-59), SEWResNet (:123-210) with the 7x7/2 stem, BN, neuron on the stem
output repeated over T (:199-202), MaxPool2d(3, 2, 1) per timestep (:143, :203), four
stages of two BasicBlocks (:145-151, :213-214), 1x1/stride downsample Conv+BN+neuron
(:172-179), AdaptiveAvgPool2d(1) per timestep (:152, :208), mean over T and Linear
(:209-210).  Parameters use the reference's state_dict key names, so a reference
checkpoint's tensors can be fed to both this restatement and the GPU engine.

Pinning: the network is a composition of functions pinned in tests/test_oracle.py
(conv_bn_seq against a float64 brute-force convolution, multistep_lif / multistep_if
against closed forms, prune_conv_2_4 against brute-force top-2); max/avg pooling, the
temporal mean and the Linear head are single torch calls checked against numpy in
tests/test_oracle_sew.py, and the block wiring (which tensor feeds which) is checked
there against hand-built expectations on tiny inputs.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .reference_path import BNParams, conv_bn_seq, multistep_if, multistep_lif, prune_conv_2_4

STAGES = ((64, 1), (128, 2), (256, 2), (512, 2))  # (planes, first stride); 2 BasicBlocks each


def conv_names():
    """(state-dict prefix of the conv weight, prefix of its BN, C_in, C_out, k, stride, pad)
    for every conv of sew_resnet18, in forward order."""
    out = [("conv1", "bn1", 3, 64, 7, 2, 3)]
    inplanes = 64
    for si, (planes, stride) in enumerate(STAGES):
        for bi in range(2):
            s = stride if bi == 0 else 1
            p = f"layer{si + 1}.{bi}"
            out.append((f"{p}.conv1.module.0", f"{p}.conv1.module.1", inplanes, planes, 3, s, 1))
            out.append((f"{p}.conv2.module.0", f"{p}.conv2.module.1", planes, planes, 3, 1, 1))
            if bi == 0 and (s != 1 or inplanes != planes):
                out.append((f"{p}.downsample.0.module.0", f"{p}.downsample.0.module.1", inplanes, planes, 1, s, 0))
            inplanes = planes
    return out


def make_params(seed: int = 0, num_classes: int = 100, in_channels: int = 3, prune: bool = True,
                bn_random: bool = False, fp16_weights: bool = False) -> dict:
    """Random parameters with the reference's initialisation (models/sewresnet.py:155-160):
    conv weights kaiming_normal(fan_out, relu), BN weight 1 / bias 0 with default running
    statistics (mean 0, var 1), Linear as nn.Linear's default (uniform +-1/sqrt(fan_in)).
    prune: 2:4 magnitude mask along C_in on every conv except the stem.
    bn_random: BN drawn as in config 0 (gamma~U(0.5,1.5)*gain ... ) to get spiking activity
    in deep layers (tests).  fp16_weights: round pruned conv weights to fp16."""
    g = torch.Generator().manual_seed(seed)
    p = {}
    for wname, bnname, cin, cout, k, _, _ in conv_names():
        if wname == "conv1":
            cin = in_channels
        std = math.sqrt(2.0 / (cout * k * k))
        w = torch.randn((cout, cin, k, k), generator=g) * std
        if prune and wname != "conv1":
            w = prune_conv_2_4(w)
        if fp16_weights and wname != "conv1":
            w = w.half().float()
        p[wname + ".weight"] = w
        if bn_random:
            p[bnname + ".weight"] = (torch.rand(cout, generator=g) + 0.5) * 2.5
            p[bnname + ".bias"] = torch.randn(cout, generator=g) * 0.3 + 0.5
            p[bnname + ".running_mean"] = torch.randn(cout, generator=g) * 0.1
            p[bnname + ".running_var"] = torch.rand(cout, generator=g) + 0.5
        else:
            p[bnname + ".weight"] = torch.ones(cout)
            p[bnname + ".bias"] = torch.zeros(cout)
            p[bnname + ".running_mean"] = torch.zeros(cout)
            p[bnname + ".running_var"] = torch.ones(cout)
    bound = 1.0 / math.sqrt(512)
    p["fc.weight"] = (torch.rand((num_classes, 512), generator=g) * 2 - 1) * bound
    p["fc.bias"] = (torch.rand(num_classes, generator=g) * 2 - 1) * bound
    return p


def _bn(p, name) -> BNParams:
    return BNParams(p[name + ".weight"], p[name + ".bias"], p[name + ".running_mean"], p[name + ".running_var"],
                    1e-5)


def _neuron(x_seq, neuron, tau, v_th, v_reset):
    if neuron == "lif":
        return multistep_lif(x_seq, tau, v_th, v_reset)[0]
    return multistep_if(x_seq, v_th, v_reset)[0]


def forward(p: dict, x: torch.Tensor, T: int = 4, neuron: str = "lif", tau: float = 2.0, v_th: float = 1.0,
            v_reset: float = 0.0, record: dict | None = None) -> torch.Tensor:
    """SEWResNet.forward for a 4-D image batch x (B, 3, H, W), fp32 on the CPU.
    record (optional) receives every spike / SEW tensor by name, (T, B, C, H, W)."""
    x = F.conv2d(x, p["conv1.weight"], None, stride=2, padding=3)                  # :199
    b = _bn(p, "bn1")
    x = F.batch_norm(x, b.mean, b.var, b.gamma, b.beta, training=False, eps=b.eps)   # :200
    x = x.unsqueeze(0).repeat(T, 1, 1, 1, 1)                                         # :201
    x = _neuron(x, neuron, tau, v_th, v_reset)                                       # :202
    if record is not None:
        record["stem"] = x
    y = F.max_pool2d(x.flatten(0, 1), 3, 2, 1)                                      # :203
    x = y.view(T, -1, *y.shape[1:])
    if record is not None:
        record["maxpool"] = x
    inplanes = 64
    for si, (planes, stride) in enumerate(STAGES):
        for bi in range(2):
            s = stride if bi == 0 else 1
            pre = f"layer{si + 1}.{bi}"
            identity = x                                                             # :51
            out = _neuron(conv_bn_seq(x, p[pre + ".conv1.module.0.weight"], _bn(p, pre + ".conv1.module.1"), s, 1),
                          neuron, tau, v_th, v_reset)                                # :52
            if record is not None:
                record[pre + ".sn1"] = out
            out = _neuron(conv_bn_seq(out, p[pre + ".conv2.module.0.weight"], _bn(p, pre + ".conv2.module.1"), 1, 1),
                          neuron, tau, v_th, v_reset)                                # :53
            if record is not None:
                record[pre + ".sn2"] = out
            if bi == 0 and (s != 1 or inplanes != planes):                           # :55-56, :172-179
                identity = _neuron(conv_bn_seq(x, p[pre + ".downsample.0.module.0.weight"],
                                               _bn(p, pre + ".downsample.0.module.1"), s, 0),
                                   neuron, tau, v_th, v_reset)
                if record is not None:
                    record[pre + ".downsample"] = identity
            x = out + identity                                                       # :58-59 (ADD)
            if record is not None:
                record[pre] = x
            inplanes = planes
    x = F.adaptive_avg_pool2d(x.flatten(0, 1), 1).view(T, x.shape[1], -1)           # :208-209
    return F.linear(x.mean(dim=0), p["fc.weight"], p["fc.bias"])                    # :210


def make_images(seed: int, B: int, H: int = 32, W: int = 32, C: int = 3) -> torch.Tensor:
    """Config-2 inputs: pixels ~ U(0, 1), direct-encoded (the same image at every t)."""
    g = torch.Generator().manual_seed(seed)
    return torch.rand((B, C, H, W), generator=g)
