"""CPU restatement of Spikformer's spiking layers — TEST INFRASTRUCTURE ONLY.

Follows models/spikformer.py of the reference:
  * Linear + BatchNorm1d + MultiStepLIF on tokens (MLP fc1/fc2, :63-70; SSA q/k/v/proj,
    :103-125): x (T, B, N, C) flattened to (T*B, N, C), nn.Linear (with bias), BN over the
    channel dim (transpose), reshape back, LIF;
  * spiking self-attention (:103-125): q, k, v spikes split into heads (T, B, H, N, d),
    attn = (q @ k^T) * scale, x = attn @ v, heads merged back to (T, B, N, C), attn_lif
    (LIF tau 2, V_th 0.5).

Pinning (tests/test_oracle_spikformer.py): the attention against explicit loops on tiny
inputs, exactness of every partial sum (integers times a power of two) shown by the two
associations (q k^T) v and q (k^T v) agreeing bit for bit, and Linear+BN against the
folded affine of reference_path.fold_batchnorm.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .reference_path import BNParams, multistep_lif


def linear_bn_lif(x: torch.Tensor, w: torch.Tensor, bias, bn: BNParams, tau=2.0, v_threshold=1.0, v_reset=0.0):
    """(T, B, N, C_in) -> spikes, membrane, BN output, each (T, B, N, C_out) (models/spikformer.py:63-70)."""
    T, B, N, _ = x.shape
    y = F.linear(x.flatten(0, 1), w, bias)                                        # (T*B, N, C_out)
    y = F.batch_norm(y.transpose(-1, -2), bn.mean, bn.var, bn.gamma, bn.beta, training=False,
                     eps=bn.eps).transpose(-1, -2)
    y = y.reshape(T, B, N, -1).contiguous()
    s, h, _ = multistep_lif(y, tau, v_threshold, v_reset)
    return s, h, y


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, heads: int, scale=0.125):
    """x before attn_lif (models/spikformer.py:110-123): (T, B, N, C) spikes -> (T, B, N, C)."""
    T, B, N, C = q.shape
    d = C // heads

    def split(t):
        return t.reshape(T, B, N, heads, d).permute(0, 1, 3, 2, 4).contiguous()

    qh, kh, vh = split(q), split(k), split(v)
    attn = (qh @ kh.transpose(-2, -1).contiguous()) * scale
    x = attn @ vh
    return x.transpose(2, 3).reshape(T, B, N, C).contiguous()


def ssa(q, k, v, heads: int, scale=0.125, tau=2.0, v_threshold=0.5, v_reset=0.0):
    """Spikes of attn_lif over the attention output, and that output."""
    x = attention(q, k, v, heads, scale)
    s, h, _ = multistep_lif(x, tau, v_threshold, v_reset)
    return s, h, x
