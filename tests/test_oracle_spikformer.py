"""Pins of the Spikformer restatement (oracle/spikformer.py) on the CPU."""
import numpy as np
import torch

from oracle import reference_path as ref
from oracle import spikformer as sf


def _spikes(shape, p, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(shape, generator=g) < p).float()


def test_attention_against_loops():
    T, B, N, C, H = 2, 1, 5, 32, 2
    q, k, v = (_spikes((T, B, N, C), 0.4, s) for s in (1, 2, 3))
    x = sf.attention(q, k, v, H, 0.125)
    d = C // H
    for t in range(T):
        for n in range(N):
            for h in range(H):
                for j in range(d):
                    acc = 0.0
                    for m in range(N):
                        a = sum(float(q[t, 0, n, h * d + i] * k[t, 0, m, h * d + i]) for i in range(d)) * 0.125
                        acc += a * float(v[t, 0, m, h * d + j])
                    assert float(x[t, 0, n, h * d + j]) == acc


def test_attention_is_exact_in_either_association():
    T, B, N, C, H = 2, 2, 300, 96, 2
    q, k, v = (_spikes((T, B, N, C), 0.3, s) for s in (4, 5, 6))
    x = sf.attention(q, k, v, H, 0.125)
    d = C // H
    qh = q.reshape(T, B, N, H, d).permute(0, 1, 3, 2, 4)
    kh = k.reshape(T, B, N, H, d).permute(0, 1, 3, 2, 4)
    vh = v.reshape(T, B, N, H, d).permute(0, 1, 3, 2, 4)
    kv = kh.transpose(-2, -1).contiguous() @ vh.contiguous()
    x2 = ((qh.contiguous() @ kv) * 0.125).transpose(2, 3).reshape(T, B, N, C)
    assert torch.equal(x, x2)
    assert torch.equal(x * 8, torch.round(x * 8))  # integers times 1/8


def test_linear_bn_matches_folded_affine():
    g = torch.Generator().manual_seed(7)
    T, B, N, Ci, Co = 2, 2, 9, 16, 24
    x = _spikes((T, B, N, Ci), 0.3, 8)
    w = torch.randn(Co, Ci, generator=g) * 0.3
    b = torch.randn(Co, generator=g) * 0.1
    bn = ref.BNParams(torch.rand(Co, generator=g) + 0.5, torch.randn(Co, generator=g) * 0.1,
                      torch.randn(Co, generator=g) * 0.1, torch.rand(Co, generator=g) + 0.5)
    _, _, y = sf.linear_bn_lif(x, w, b, bn)
    sc, bi = ref.fold_batchnorm(bn.gamma, bn.beta, bn.mean, bn.var, bn.eps, b)
    y2 = (x @ w.T) * torch.from_numpy(sc) + torch.from_numpy(bi)
    assert torch.allclose(y, y2, atol=1e-5)


# ---- the whole network (oracle/spikformer.py forward / sps / block)

def _small_params(seed=0):
    return sf.make_params(seed, embed=128, depth=2, num_classes=10)


def test_params_use_reference_names_and_are_2_4():
    p = sf.make_params(0, embed=384, depth=8, init="reference")
    assert p["patch_embed.proj_conv.weight"].shape == (48, 3, 3, 3)
    assert p["patch_embed.rpe_conv.weight"].shape == (384, 384, 3, 3)
    assert p["block.7.mlp.fc1_linear.weight"].shape == (1536, 384)
    assert p["head.weight"].shape == (1000, 384)
    for name in ("patch_embed.proj_conv1.weight", "patch_embed.rpe_conv.weight"):
        assert ref.verify_n_m(ref.conv_weight_2d(p[name]))
    for name in ("block.0.attn.q_linear.weight", "block.3.mlp.fc2_linear.weight"):
        assert ref.verify_n_m(p[name])
    assert bool((p["patch_embed.proj_conv.weight"] != 0).all())  # C_in = 3 stays dense


def _never(p, bn):  # BN bias far below threshold: the layer never fires
    p[bn + ".bias"] = torch.full_like(p[bn + ".bias"], -1e4)


def _always(p, bn):  # BN bias far above threshold: the layer fires at every step
    p[bn + ".bias"] = torch.full_like(p[bn + ".bias"], 1e4)


def test_sps_adds_rpe_spikes_to_pooled_features():
    p = _small_params()
    x = torch.randn(2, 3, 16, 16, generator=torch.Generator().manual_seed(1)).unsqueeze(0).repeat(4, 1, 1, 1, 1)
    rec = {}
    _never(p, "patch_embed.rpe_bn")
    y = sf.sps(p, x, rec)
    feat = rec["x_feat"]
    assert torch.equal(y, feat.flatten(-2).transpose(-1, -2))  # rpe silent: tokens = pooled features
    _always(p, "patch_embed.rpe_bn")
    y = sf.sps(p, x, rec)
    assert torch.equal(y, feat.flatten(-2).transpose(-1, -2) + 1.0)
    # the max-pools: 3x3 / 2 / pad 1 of the third and fourth stages' spikes
    s3 = rec["proj_conv3"]
    exp = torch.nn.functional.max_pool2d(s3.flatten(0, 1), 3, 2, 1).view_as(feat)
    assert torch.equal(feat, exp)
    assert y.shape == (4, 2, 16, 128) and float(rec["proj_conv"].mean()) > 0.01


def test_block_adds_attention_then_mlp_spikes():
    p = _small_params()
    g = torch.Generator().manual_seed(2)
    x = torch.randint(0, 3, (4, 2, 10, 128), generator=g).float()
    q = dict(p)
    _never(q, "block.0.attn.proj_bn")
    _never(q, "block.0.mlp.fc2_bn")
    assert torch.equal(sf.block(q, "block.0", x, 2), x)  # both branches silent: identity
    _always(q, "block.0.attn.proj_bn")
    assert torch.equal(sf.block(q, "block.0", x, 2), x + 1.0)  # attention branch adds its spikes
    _never(q, "block.0.attn.proj_bn")
    _always(q, "block.0.mlp.fc2_bn")
    assert torch.equal(sf.block(q, "block.0", x, 2), x + 1.0)  # MLP branch adds its spikes
    rec = {}
    out = sf.block(p, "block.0", x, 2, rec)
    assert set(torch.unique(out - rec["block.0.attn"]).tolist()) <= {0.0, 1.0}
    assert set(torch.unique(rec["block.0.attn"] - x).tolist()) <= {0.0, 1.0}


def test_forward_head_is_token_then_time_mean_then_linear():
    p = _small_params()
    x = torch.randn(2, 3, 16, 16, generator=torch.Generator().manual_seed(3))
    logits, xs = sf.forward(p, x, T=4, heads=2, depth=2, keep=True)
    feat = xs[-1].double().numpy().mean(axis=2).mean(axis=0)
    exp = feat @ p["head.weight"].double().numpy().T + p["head.bias"].double().numpy()
    assert np.allclose(logits.double().numpy(), exp, atol=1e-5)
    assert len(xs) == 3 and float(xs[-1].max()) <= 6  # 2 after SPS + 2 per block
