"""2:4 weight preparation and BatchNorm folding (host side, torch/numpy).

Mirrors the reference's offline weight preparation:
  * prune_n_m / prune_2_4 / verify_n_m  — sparse/pruning.py:28-118
  * conv_weight_2d / conv_weight_back   — sparse/utils.py:87-120 (2:4 along C_in per (k, r, s))
  * validate_2_4_pattern                — sengine/optimizer.py:499-523
  * fold_batchnorm                      — sengine/optimizer.py:126-191 (float64 fold, fp32 storage)
These run once per node at build time; they work on CPU or GPU tensors.
"""
from __future__ import annotations

from functools import partial

import numpy as np
import torch


def prune_n_m(weight: torch.Tensor, n: int = 2, m: int = 4) -> torch.Tensor:
    """Zero the (m-n) smallest-|w| entries of every m-group along the last dim (the last dim
    is zero-padded to a multiple of m for grouping).  Same rule and tie handling as
    sparse/pruning.py:28-76 (torch.topk(largest=False) picks the entries to drop)."""
    if not 0 < n < m:
        raise ValueError(f"need 0 < n < m, got n={n}, m={m}")
    shape, dtype = weight.shape, weight.dtype
    rows = weight.reshape(-1, shape[-1])
    cols = rows.shape[1]
    pad = (-cols) % m
    if pad:
        rows = torch.nn.functional.pad(rows, (0, pad))
    g = rows.reshape(rows.shape[0], -1, m)
    drop = g.abs().topk(m - n, dim=2, largest=False).indices
    keep = torch.ones_like(g).scatter_(2, drop, 0.0)
    out = (g * keep).reshape(rows.shape[0], -1)[:, :cols]
    return out.reshape(shape).to(dtype)


prune_2_4 = partial(prune_n_m, n=2, m=4)


def verify_n_m(weight: torch.Tensor, n: int = 2, m: int = 4) -> bool:
    """True when every full m-group along dim 1 of a 2-D tensor has exactly m-n zeros."""
    if weight.ndim != 2:
        return False
    width = (weight.shape[1] // m) * m
    if width == 0:
        return True
    g = weight[:, :width].reshape(weight.shape[0], width // m, m)
    return bool(((g == 0).sum(dim=2) == m - n).all().item())


verify_2_4 = partial(verify_n_m, n=2, m=4)


def conv_weight_2d(w: torch.Tensor) -> torch.Tensor:
    """(K, C, R, S) -> (K*R*S, C)."""
    K, C, R, S = w.shape
    return w.permute(0, 2, 3, 1).reshape(K * R * S, C).contiguous()


def conv_weight_back(w2d: torch.Tensor, shape) -> torch.Tensor:
    K, C, R, S = shape
    return w2d.reshape(K, R, S, C).permute(0, 3, 1, 2).contiguous()


def prune_conv_2_4(w: torch.Tensor) -> torch.Tensor:
    """2:4 magnitude pruning of a conv weight along input channels."""
    return conv_weight_back(prune_2_4(conv_weight_2d(w)), w.shape)


def validate_2_4_pattern(weight) -> bool:
    """Engine 2:4 check: conv weights viewed as (K, R*S*C); every 4-group must contain
    exactly two entries with |w| < 1e-10."""
    w = weight.detach().cpu().numpy() if isinstance(weight, torch.Tensor) else np.asarray(weight)
    if w.ndim == 4:
        flat = w.transpose(0, 2, 3, 1).reshape(w.shape[0], -1)
    elif w.ndim == 2:
        flat = w
    else:
        return False
    rows, cols = flat.shape
    if cols < 4 or cols % 4:
        return False
    zeros = (np.abs(flat.reshape(rows, cols // 4, 4)) < 1e-10).sum(axis=2)
    return bool((zeros == 2).all())


def fold_batchnorm(gamma, beta, running_mean, running_var, eps: float = 1e-5, conv_bias=None):
    """Eval BatchNorm -> per-channel (scale, bias) for the epilogue y = acc*scale + bias:
    scale = gamma / sqrt(var + eps), bias = scale * (b - mean) + beta, in float64, stored fp32."""
    def f64(x):
        return (x.detach().cpu().double().numpy() if isinstance(x, torch.Tensor)
                else np.asarray(x, dtype=np.float64))
    g, b, mu, var = f64(gamma), f64(beta), f64(running_mean), f64(running_var)
    scale = g * (1.0 / np.sqrt(var + eps))
    cb = np.zeros_like(mu) if conv_bias is None else f64(conv_bias)
    bias = scale * (cb - mu) + b
    return torch.from_numpy(scale.astype(np.float32)), torch.from_numpy(bias.astype(np.float32))


def expand_planes(w: torch.Tensor, planes: int) -> torch.Tensor:
    """Weights for a conv whose input is stored as `planes` bit planes (an integer activation
    x = sum_p 2^p b_p, e.g. a SEW 'ADD' output): conv(x, W) = conv([b_0, b_1, ...], [W, 2W, ...])
    with the planes stacked along the input channels.  Scaling by 2^p is exact in fp16/fp32 and
    keeps the 2:4 pattern of every plane's copy."""
    return torch.cat([w * float(1 << p) for p in range(planes)], dim=1)
