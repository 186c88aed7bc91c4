"""Pins of the Spikformer restatement (oracle/spikformer.py) on the CPU."""
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
