"""CPU restatement of Spikformer's spiking layers — TEST INFRASTRUCTURE ONLY.

Follows models/spikformer.py of the reference:
  * Linear + BatchNorm1d + MultiStepLIF on tokens (MLP fc1/fc2, :63-70; SSA q/k/v/proj,
    :103-125): x (T, B, N, C) flattened to (T*B, N, C), nn.Linear (with bias), BN over the
    channel dim (transpose), reshape back, LIF;
  * spiking self-attention (:103-125): q, k, v spikes split into heads (T, B, H, N, d),
    attn = (q @ k^T) * scale, x = attn @ v, heads merged back to (T, B, N, C), attn_lif
    (LIF tau 2, V_th 0.5).

  * the whole network (forward, :250-288): SPS patch splitting (:160-209: four 3x3
    Conv+BN+LIF stages on the T-repeated image, max-pools after the third and fourth, the
    relative-position conv whose LIF spikes are added to the max-pooled features), eight
    Blocks (:138-150: x = x + SSA(x); x = x + MLP(x) -- an integer-valued residual stream),
    mean over tokens, mean over T, Linear head.

Pinning (tests/test_oracle_spikformer.py): the attention against explicit loops on tiny
inputs, exactness of every partial sum (integers times a power of two) shown by the two
associations (q k^T) v and q (k^T v) agreeing bit for bit, and Linear+BN against the
folded affine of reference_path.fold_batchnorm; the SPS wiring, the block's two residual
adds and the head on hand-built special cases (zeroed layers whose output is known).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

import math

from .reference_path import BNParams, conv_bn_seq, multistep_lif, prune_conv_2_4


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


# --------------------------------------------------------------------------------------
# The whole network (models/spikformer.py:153-288)
# --------------------------------------------------------------------------------------

def sps_channels(embed: int):
    """(name, C_in, C_out) of the SPS convs (:167-185): embed/8, /4, /2, embed, rpe."""
    return [("proj_conv", None, embed // 8), ("proj_conv1", embed // 8, embed // 4),
            ("proj_conv2", embed // 4, embed // 2), ("proj_conv3", embed // 2, embed), ("rpe_conv", embed, embed)]


def _bn_name(conv: str) -> str:
    return conv.replace("conv", "bn")


def make_params(seed: int = 0, embed: int = 384, depth: int = 8, mlp_ratio: int = 4, num_classes: int = 1000,
                in_channels: int = 3, init: str = "lively", fp16_weights: bool = True) -> dict:
    """Random Spikformer parameters keyed by the reference's state_dict names
    (patch_embed.proj_conv.weight, patch_embed.proj_bn.*, block.{i}.attn.q_linear.*, ...,
    block.{i}.mlp.fc2_bn.*, head.*).  Every conv but the first (C_in = 3) and every Linear
    of the blocks is 2:4-pruned along its input, rounded to fp16 when
    fp16_weights.  init='reference': the model's own _init_weights (:238-245: Linear
    truncated N(0, 0.02), bias 0; conv and BN PyTorch defaults); init='lively': conv and
    Linear N(0, 2/fan_in) (times 1/sqrt(0.15) where the input is spikes) and BN drawn as in
    config 0, so that every layer spikes."""
    g = torch.Generator().manual_seed(seed)
    p = {}

    def wdraw(shape, fan_in, linear):
        if init == "reference":
            if linear:
                return (torch.randn(shape, generator=g) * 0.02).clamp_(-0.04, 0.04)
            b = 1.0 / math.sqrt(fan_in)
            return (torch.rand(shape, generator=g) * 2 - 1) * b
        # spike inputs fire at ~15%: scale so the pre-BN output has about unit variance
        gain = 1.0 if (not linear and fan_in == in_channels * 9) else 1.0 / math.sqrt(0.15)
        return torch.randn(shape, generator=g) * math.sqrt(2.0 / fan_in) * gain

    def prune(w):
        w = prune_conv_2_4(w if w.ndim == 4 else w[:, :, None, None])
        w = w.half().float() if fp16_weights else w
        return w

    def bn(name, c):
        if init == "reference":
            p[name + ".weight"], p[name + ".bias"] = torch.ones(c), torch.zeros(c)
            p[name + ".running_mean"], p[name + ".running_var"] = torch.zeros(c), torch.ones(c)
        else:
            p[name + ".weight"] = torch.rand(c, generator=g) + 0.5
            p[name + ".bias"] = torch.randn(c, generator=g) * 0.1
            p[name + ".running_mean"] = torch.randn(c, generator=g) * 0.1
            p[name + ".running_var"] = torch.rand(c, generator=g) + 0.5

    for name, cin, cout in sps_channels(embed):
        cin = in_channels if cin is None else cin
        w = wdraw((cout, cin, 3, 3), cin * 9, False)
        p[f"patch_embed.{name}.weight"] = w if name == "proj_conv" else prune(w)
        bn(f"patch_embed.{_bn_name(name)}", cout)
    hidden = embed * mlp_ratio
    for i in range(depth):
        pre = f"block.{i}"
        for lin, cin, cout in (("attn.q", embed, embed), ("attn.k", embed, embed), ("attn.v", embed, embed),
                               ("attn.proj", embed, embed), ("mlp.fc1", embed, hidden), ("mlp.fc2", hidden, embed)):
            p[f"{pre}.{lin}_linear.weight"] = prune(wdraw((cout, cin), cin, True))[:, :, 0, 0]
            p[f"{pre}.{lin}_linear.bias"] = torch.zeros(cout) if init == "reference" else \
                torch.randn(cout, generator=g) * 0.1
            bn(f"{pre}.{lin}_bn", cout)
    p["head.weight"] = wdraw((num_classes, embed), embed, True) if init == "reference" else \
        torch.randn(num_classes, embed, generator=g) * 0.05
    p["head.bias"] = torch.zeros(num_classes) if init == "reference" else torch.randn(num_classes, generator=g) * 0.1
    return p


def bn_of(p: dict, name: str) -> BNParams:
    return BNParams(p[name + ".weight"], p[name + ".bias"], p[name + ".running_mean"], p[name + ".running_var"], 1e-5)


def sps(p: dict, x_seq: torch.Tensor, record: dict | None = None) -> torch.Tensor:
    """SPS.forward (:187-209) on (T, B, C, H, W) -> tokens (T, B, N, embed), integer-valued
    (rpe spikes + max-pooled features)."""
    def stage(x, name):
        y = conv_bn_seq(x, p[f"patch_embed.{name}.weight"], bn_of(p, f"patch_embed.{_bn_name(name)}"), 1, 1)
        s = multistep_lif(y)[0]
        if record is not None:
            record[name] = s
        return s

    def pool(x):
        T = x.shape[0]
        y = F.max_pool2d(x.flatten(0, 1), kernel_size=3, stride=2, padding=1)
        return y.view(T, -1, *y.shape[1:])

    x = stage(x_seq, "proj_conv")
    x = stage(x, "proj_conv1")
    x = pool(stage(x, "proj_conv2"))
    x_feat = pool(stage(x, "proj_conv3"))
    if record is not None:
        record["x_feat"] = x_feat
    x = stage(x_feat, "rpe_conv") + x_feat
    T, B, C, H, W = x.shape
    return x.flatten(-2).transpose(-1, -2)  # (T, B, N, C)


def block(p: dict, pre: str, x: torch.Tensor, heads: int, record: dict | None = None) -> torch.Tensor:
    """Block.forward (:147-150): x = x + SSA(x) (:103-135); x = x + MLP(x) (:59-70)."""
    def lin(name, inp, v_th=1.0):
        return linear_bn_lif(inp, p[f"{pre}.{name}_linear.weight"], p[f"{pre}.{name}_linear.bias"],
                             bn_of(p, f"{pre}.{name}_bn"), 2.0, v_th)[0]

    q, k, v = lin("attn.q", x), lin("attn.k", x), lin("attn.v", x)
    a = ssa(q, k, v, heads)[0]
    x = x + lin("attn.proj", a)
    if record is not None:
        record[pre + ".attn"] = x
    h = lin("mlp.fc1", x)
    x = x + lin("mlp.fc2", h)
    return x


def forward(p: dict, x_img: torch.Tensor, T: int = 4, heads: int = 8, depth: int = 8, keep: bool = False):
    """Spikformer.forward (:281-288) for images (B, C, H, W): the image repeated over T, SPS,
    the blocks, mean over tokens (:277-279) and T, Linear.  keep=True also returns the
    token stream before each block and after the last."""
    with torch.no_grad():
        x = sps(p, x_img.float().unsqueeze(0).repeat(T, 1, 1, 1, 1))
        xs = [x]
        for i in range(depth):
            x = block(p, f"block.{i}", x, heads)
            xs.append(x)
        logits = F.linear(x.mean(2).mean(0), p["head.weight"], p["head.bias"])
    return (logits, xs) if keep else logits
