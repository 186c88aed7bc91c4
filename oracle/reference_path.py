"""Restatement of the SparseSNN reference PyTorch path for one fused layer (CPU, fp32).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Every function cites the
reference file:line it follows.  The arithmetic is done with the same torch ops in
the same order as the reference, so it reproduces the reference's CPU results.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F


# --------------------------------------------------------------------------------------
# 2:4 pruning (sparse/pruning.py:28-118, sparse/utils.py:87-120)
# --------------------------------------------------------------------------------------

def prune_n_m(weight: torch.Tensor, n: int = 2, m: int = 4) -> torch.Tensor:
    """Magnitude N:M pruning along the last dim — sparse/pruning.py:28-76.

    Each group of m consecutive elements keeps its n largest |w|: the (m-n) smallest
    are found with topk(largest=False) and zeroed through a scattered mask; the last
    dim is zero-padded to a multiple of m and the padding dropped afterwards.
    """
    assert 0 < n < m
    shape, dtype = weight.shape, weight.dtype
    w2d = weight.reshape(-1, shape[-1])
    rows, cols = w2d.shape
    pad = (m - cols % m) % m
    if pad:
        w2d = torch.cat([w2d, torch.zeros(rows, pad, dtype=dtype, device=w2d.device)], dim=1)
    grouped = w2d.reshape(rows, w2d.shape[1] // m, m)
    _, small = grouped.abs().topk(m - n, dim=2, largest=False)
    mask = torch.ones_like(grouped)
    mask.scatter_(2, small, 0.0)
    out = (grouped * mask).reshape(rows, -1)
    if pad:
        out = out[:, :cols]
    return out.reshape(shape)


def conv_weight_2d(w: torch.Tensor) -> torch.Tensor:
    """Conv weight (K, C, R, S) -> (K*R*S, C): 2:4 runs along C for each (k, r, s).
    sparse/utils.py:87-109 (_get_weight_2d)."""
    K, C, R, S = w.shape
    return w.permute(0, 2, 3, 1).reshape(K * R * S, C).contiguous()


def conv_weight_back(w2d: torch.Tensor, shape) -> torch.Tensor:
    """Inverse of conv_weight_2d — sparse/utils.py:112-120 (_write_weight_back)."""
    K, C, R, S = shape
    return w2d.reshape(K, R, S, C).permute(0, 3, 1, 2).contiguous()


def prune_conv_2_4(w: torch.Tensor) -> torch.Tensor:
    """2:4 along input channels of a conv weight, as the reference prunes conv layers."""
    return conv_weight_back(prune_n_m(conv_weight_2d(w), 2, 4), w.shape)


def verify_n_m(weight: torch.Tensor, n: int = 2, m: int = 4) -> bool:
    """Every full group of m along dim 1 has exactly m-n zeros — sparse/pruning.py:91-115."""
    if weight.ndim != 2:
        return False
    rows, cols = weight.shape
    width = (cols // m) * m
    if width == 0:
        return True
    grouped = weight[:, :width].reshape(rows, width // m, m)
    return bool(((grouped == 0).sum(dim=2) == m - n).all().item())


def validate_2_4_pattern(weight: np.ndarray) -> bool:
    """Engine-side 2:4 check — sengine/optimizer.py:499-523: conv (K,C,R,S) viewed as
    (K, R*S*C); each 4-group must have exactly two entries with |w| < 1e-10."""
    if weight.ndim == 4:
        flat = weight.transpose(0, 2, 3, 1).reshape(weight.shape[0], -1)
    elif weight.ndim == 2:
        flat = weight
    else:
        return False
    rows, cols = flat.shape
    if cols < 4 or cols % 4 != 0:
        return False
    zeros = np.sum(np.abs(flat.reshape(rows, cols // 4, 4)) < 1e-10, axis=2)
    return bool(np.all(zeros == 2))


# --------------------------------------------------------------------------------------
# BatchNorm (eval) and its engine fold (sengine/optimizer.py:126-191)
# --------------------------------------------------------------------------------------

def fold_batchnorm(gamma, beta, mean, var, eps=1e-5, conv_bias=None):
    """scale = gamma/sqrt(var+eps), bias = scale*(b - mean) + beta, both computed in float64
    and stored as float32 — sengine/optimizer.py:159-183.  Weights are not scaled (:168-171)."""
    g = np.asarray(gamma, np.float64)
    b_ = np.asarray(beta, np.float64)
    mu = np.asarray(mean, np.float64)
    v = np.asarray(var, np.float64)
    scale = g * (1.0 / np.sqrt(v + eps))
    cb = np.zeros_like(mu) if conv_bias is None else np.asarray(conv_bias, np.float64)
    bias = scale * (cb - mu) + b_
    return scale.astype(np.float32), bias.astype(np.float32)


@dataclass
class BNParams:
    gamma: torch.Tensor
    beta: torch.Tensor
    mean: torch.Tensor
    var: torch.Tensor
    eps: float = 1e-5


def conv_bn_seq(x_seq: torch.Tensor, w: torch.Tensor, bn: BNParams, stride=1, padding=0,
                dilation=1) -> torch.Tensor:
    """SeqToANNContainer(Conv2d(bias=False), BatchNorm2d) in eval mode:
    flatten (T, B) -> conv -> BN -> view back (models/layers.py:26-31,
    models/sewresnet.py:18-24,37-40)."""
    T = x_seq.shape[0]
    y = F.conv2d(x_seq.flatten(0, 1), w, None, stride=stride, padding=padding, dilation=dilation)
    y = F.batch_norm(y, bn.mean, bn.var, bn.gamma, bn.beta, training=False, eps=bn.eps)
    return y.view(T, -1, *y.shape[1:])


# --------------------------------------------------------------------------------------
# Multi-step neurons (models/neurons.py:121-146,169-184,205-231)
# --------------------------------------------------------------------------------------

def multistep_lif(x_seq: torch.Tensor, tau=2.0, v_threshold=1.0, v_reset=0.0, v0=None):
    """MultiStepLIFNeuron.forward: V reset to 0 at each call (neurons.py:205-211), then per t
    charge v = v*(1-1/tau) + x/tau (:124), fire (v - v_th).ge(0) (:127, :41), reset
    hard v=(1-s)v + s*v_reset or soft v = v - s*v_th (v_reset None) (:129-140).
    Returns (spikes, charged membrane h per t)."""
    v = torch.zeros_like(x_seq[0]) if v0 is None else v0.clone()
    spikes, hs = [], []
    for t in range(x_seq.shape[0]):
        v = v * (1.0 - 1.0 / tau) + x_seq[t] / tau
        hs.append(v)
        s = (v - v_threshold).ge(0.0).to(x_seq.dtype)
        if v_reset is None:
            v = v - s * v_threshold
        else:
            v = (1.0 - s) * v + s * v_reset
        spikes.append(s)
    return torch.stack(spikes, 0), torch.stack(hs, 0), v


def multistep_if(x_seq: torch.Tensor, v_threshold=1.0, v_reset=0.0, v0=None):
    """MultiStepIFNeuron.forward: v = v + x (neurons.py:169-172), same fire/reset (:173-183)."""
    v = torch.zeros_like(x_seq[0]) if v0 is None else v0.clone()
    spikes, hs = [], []
    for t in range(x_seq.shape[0]):
        v = v + x_seq[t]
        hs.append(v)
        s = (v - v_threshold).ge(0.0).to(x_seq.dtype)
        if v_reset is None:
            v = v - s * v_threshold
        else:
            v = (1.0 - s) * v + s * v_reset
        spikes.append(s)
    return torch.stack(spikes, 0), torch.stack(hs, 0), v


def ms_neuron(x_seq: torch.Tensor, decay=0.25, thresh=0.5, v0=None):
    """MSNeuron.forward (models/msresnet.py:28-56): per t, mem = mem * decay * (1 - spike) + x[t]
    then spike = heaviside(mem - thresh, 'gate') = (mem - thresh).ge(0) (models/neurons.py:52-59).
    mem starts at 0 (or v0).  Returns (spikes, mem per t, mem * (1 - last spike))."""
    mem = torch.zeros_like(x_seq[0]) if v0 is None else v0.clone()
    spike = torch.zeros_like(x_seq[0])
    spikes, hs = [], []
    for t in range(x_seq.shape[0]):
        mem = mem * decay * (1.0 - spike) + x_seq[t]
        hs.append(mem)
        spike = (mem - thresh).ge(0.0).to(x_seq.dtype)
        spikes.append(spike)
    return torch.stack(spikes, 0), torch.stack(hs, 0), mem * (1.0 - spike)


def _neuron(x, neuron, tau, v_threshold, v_reset, v0):
    if neuron == "lif":
        return multistep_lif(x, tau, v_threshold, v_reset, v0)
    if neuron == "ms":  # tau carries the decay, as in the C ABI
        return ms_neuron(x, tau, v_threshold, v0)
    return multistep_if(x, v_threshold, v_reset, v0)


@dataclass
class LayerResult:
    spikes: torch.Tensor   # (T, B, C_out, OH, OW) {0,1} fp32
    h: torch.Tensor        # (T, B, C_out, OH, OW) charged membrane per t
    x: torch.Tensor        # (T, B, C_out, OH, OW) BN output (neuron input current)
    v_final: torch.Tensor  # (B, C_out, OH, OW) membrane after the last reset


def fused_layer(x_seq, w, bn: BNParams, stride=1, padding=1, dilation=1, neuron="lif", tau=2.0,
                v_threshold=1.0, v_reset=0.0, v0=None) -> LayerResult:
    """The reference PyTorch path of one fused node: Conv -> BN -> multi-step neuron.
    x_seq (T, B, C_in, H, W) fp32; w (C_out, C_in, KH, KW) fp32 (already 2:4 pruned)."""
    x = conv_bn_seq(x_seq, w, bn, stride, padding, dilation)
    s, h, v = _neuron(x, neuron, tau, v_threshold, v_reset, v0)
    return LayerResult(s, h, x, v)


def shortcut_layer(x_seq, w, bn: BNParams, residual, stride=1, padding=1, neuron="ms", tau=0.25,
                   v_threshold=0.5, v_reset=0.0, v0=None) -> LayerResult:
    """MS-ResNet's membrane shortcut around a conv: y = TDBN(conv(spikes)) + residual
    (BasicBlock18.forward, models/msresnet.py:107-112; TDBNContainer :58-80 is Conv2d on the
    flattened (T*B) batch then a per-channel eval BatchNorm), then the next neuron on y
    (the following block's sn1, :108).  Returns the neuron's result with x = y."""
    y = conv_bn_seq(x_seq, w, bn, stride, padding)
    if residual is not None:
        y = y + residual
    s, h, v = _neuron(y, neuron, tau, v_threshold, v_reset, v0)
    return LayerResult(s, h, y, v)


# --------------------------------------------------------------------------------------
# Synthetic inputs with the draw order of BASELINE.json configs 0/1
# --------------------------------------------------------------------------------------

@dataclass
class LayerCase:
    x_seq: torch.Tensor    # (T, B, C_in, H, W) fp32 {0,1}
    w: torch.Tensor        # (C_out, C_in, KH, KW) fp32, 2:4 pruned (fp16-rounded if fp16)
    bn: BNParams
    stride: int
    padding: int


def make_layer_case(seed, T, B, C_in, C_out, H, W, k, stride=1, padding=None, p_spike=0.15,
                    fp16_weights=False) -> LayerCase:
    """Seeded draw, fixed order: spikes ~ Bernoulli(p), W ~ N(0, 2/(k*k*C_in)), 2:4 mask on
    fp32 W, [fp16 round], gamma ~ U(0.5,1.5), beta ~ N(0,0.1), mean ~ N(0,0.1), var ~ U(0.5,1.5)."""
    if padding is None:
        padding = k // 2
    g = torch.Generator().manual_seed(seed)
    x = torch.bernoulli(torch.full((T, B, C_in, H, W), p_spike), generator=g)
    std = (2.0 / (k * k * C_in)) ** 0.5
    w = torch.randn((C_out, C_in, k, k), generator=g) * std
    w = prune_conv_2_4(w)
    if fp16_weights:
        w = w.half().float()
    gamma = torch.rand(C_out, generator=g) + 0.5
    beta = torch.randn(C_out, generator=g) * 0.1
    mean = torch.randn(C_out, generator=g) * 0.1
    var = torch.rand(C_out, generator=g) + 0.5
    return LayerCase(x, w, BNParams(gamma, beta, mean, var, 1e-5), stride, padding)
