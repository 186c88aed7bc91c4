"""GPU parity of the Spikformer pieces against oracle/spikformer.py:
spiking self-attention (bit-exact: the attention output is exact in fp32) and the
Linear+BN+LIF token layers run as fused 1x1 convolutions."""
import numpy as np
import pytest
import torch

from oracle import packing as pk
from oracle import reference_path as ref
from oracle import spikformer as sf
from sparsesnn_amd import ops
from sparsesnn_amd.sparsity import fold_batchnorm, prune_conv_2_4
from tests.parity import compare

pytestmark = pytest.mark.gpu


def _spikes(shape, p, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(shape, generator=g) < p).float()


def _bits(x):  # (T, B, N, C) {0,1} -> int32 (T*B, N, C/32) in the library's channel-bit order
    T, B, N, C = x.shape
    return torch.from_numpy(pk.pack_bits(x.reshape(-1, C).numpy()).view(np.int32).reshape(T * B, N, C // 32))


def _unbits(w, T, B, N, C):
    return pk.unpack_bits(w.cpu().numpy().view(np.uint32).reshape(-1, C // 32), C).reshape(T, B, N, C)


@pytest.mark.parametrize("T,B,N,C,heads,p", [(4, 2, 200, 384, 8, 0.15), (4, 1, 3136, 384, 8, 0.2),
                                             (2, 3, 70, 256, 8, 0.3), (4, 2, 130, 128, 2, 0.25),
                                             (2, 2, 65, 64, 4, 0.4), (8, 1, 100, 128, 2, 0.3), (1, 2, 90, 384, 12, 0.3),
                                             # an odd head count (one head per K^T V workgroup)
                                             (2, 2, 150, 160, 5, 0.3), (4, 1, 100, 64, 1, 0.3)])
def test_ssa_bit_exact(dev, T, B, N, C, heads, p):
    q, k, v = (_spikes((T, B, N, C), p, s) for s in (11, 12, 13))
    out = ops.spiking_self_attention(_bits(q).to(dev), _bits(k).to(dev), _bits(v).to(dev), T, B, N, C, heads)
    torch.cuda.synchronize()
    s_ref, _, x = sf.ssa(q, k, v, heads)
    got = _unbits(out, T, B, N, C)
    assert float(s_ref.mean()) > 0.01
    assert np.array_equal(got, s_ref.numpy()), int((got != s_ref.numpy()).sum())


def test_ssa_large_kv_entries(dev):
    """K^T V entries of 2048 and more (channels set together in over 2048 tokens) take the
    attend kernel's two-piece path; entries below 2048 the one-piece path.  Both bit-exact."""
    T, B, N, C, heads = 2, 1, 2200, 128, 2
    q, k, v = (_spikes((T, B, N, C), 0.3, s) for s in (31, 32, 33))
    k[:, :, :, :4] = 1.0
    v[:, :, :, 2:6] = 1.0  # head 0: KV[0..3][2..5] = 2200; head 1 keeps entries below 2048
    out = ops.spiking_self_attention(_bits(q).to(dev), _bits(k).to(dev), _bits(v).to(dev), T, B, N, C, heads)
    torch.cuda.synchronize()
    s_ref, _, x = sf.ssa(q, k, v, heads)
    got = _unbits(out, T, B, N, C)
    assert float(s_ref.mean()) > 0.01
    assert np.array_equal(got, s_ref.numpy()), int((got != s_ref.numpy()).sum())


def test_ssa_kv_workspace_matches_kt_v(dev):
    T, B, N, C, H = 2, 2, 333, 384, 8
    q, k, v = (_spikes((T, B, N, C), 0.2, s) for s in (21, 22, 23))
    kv = torch.empty(T * B, H, 48, 48, dtype=torch.int32, device=dev)
    ops.spiking_self_attention(_bits(q).to(dev), _bits(k).to(dev), _bits(v).to(dev), T, B, N, C, H, kv=kv)
    kh = k.reshape(T * B, N, H, 48).permute(0, 2, 3, 1)
    vh = v.reshape(T * B, N, H, 48).permute(0, 2, 1, 3)
    assert torch.equal(kv.cpu().float(), kh @ vh)


def test_ssa_rejects_bad_shapes(dev):
    z = torch.zeros(2 * 10 * 3, dtype=torch.int32, device=dev)
    with pytest.raises(ops.SEngineError):  # head dim 24 is not a multiple of 16
        ops.spiking_self_attention(z, z, z, 2, 1, 10, 96, 4)
    z2 = torch.zeros(2 * 10 * 12, dtype=torch.int32, device=dev)
    with pytest.raises(ops.SEngineError):  # scale must be a power of two
        ops.spiking_self_attention(z2, z2, z2, 2, 1, 10, 384, 8, scale=0.1)


@pytest.mark.parametrize("neuron,xs", [("lif", 0.25), ("if", 0.5)])  # xscale = scale * xs (LIF folds 1/tau)
def test_ssa_scale_range(dev, neuron, xs):
    """The attention's fp16 pieces are exact only for N * xscale <= 65504 and xscale >= 2^-24:
    scales at the bounds run (bit-exact against the oracle), one step past them is refused."""
    T, B, N, C, heads = 1, 1, 2048, 64, 4
    q, k, v = (_spikes((T, B, N, C), 0.9, s) for s in (31, 32, 33))
    qb, kb, vb = (_bits(a).to(dev) for a in (q, k, v))
    top = 2.0 ** int(np.floor(np.log2(65504.0 / N / xs)))  # largest power of two in range
    bottom = 2.0 ** -24 / xs
    for scale in (top, bottom):
        out = ops.spiking_self_attention(qb, kb, vb, T, B, N, C, heads, scale=scale, neuron=neuron)
        torch.cuda.synchronize()
        if neuron == "lif":
            s_ref = sf.ssa(q, k, v, heads, scale=scale)[0]
            assert np.array_equal(_unbits(out, T, B, N, C), s_ref.numpy())
    for scale in (top * 2, bottom / 2):
        with pytest.raises(ops.SEngineError, match="scale out of range"):
            ops.spiking_self_attention(qb, kb, vb, T, B, N, C, heads, scale=scale, neuron=neuron)


@pytest.mark.parametrize("N,C_in,C_out", [(197, 384, 384), (196, 384, 1536), (50, 1536, 384)])
def test_linear_bn_lif_as_fused_1x1(dev, N, C_in, C_out):
    """Spikformer's Linear (with bias) + BN1d + LIF on tokens = the fused 1x1 conv over the
    (T*B, N, 1, C) token grid, the Linear bias folded into the BN affine."""
    T, B = 4, 2
    g = torch.Generator().manual_seed(N + C_out)
    x = _spikes((T, B, N, C_in), 0.2, N)
    w = prune_conv_2_4((torch.randn(C_out, C_in, 1, 1, generator=g) * (2.0 / C_in) ** 0.5)).half().float()
    bias = torch.randn(C_out, generator=g) * 0.1
    bn = ref.BNParams((torch.rand(C_out, generator=g) + 0.5) * 3.0, torch.randn(C_out, generator=g) * 0.3 + 0.3,
                      torch.randn(C_out, generator=g) * 0.1, torch.rand(C_out, generator=g) + 0.5)
    s_ref, h_ref, _ = sf.linear_bn_lif(x, w[:, :, 0, 0], bias, bn)
    spec = ops.ConvSpec(T=T, B=B, C_in=C_in, H=N, W=1, C_out=C_out, KH=1, KW=1, padding=0)
    values, meta, _ = ops.compress_2_4(spec, w.half().to(dev))
    sc, bi = fold_batchnorm(bn.gamma, bn.beta, bn.mean, bn.var, 1e-5, bias)
    out = ops.fused_sparse_conv_bn_lif(spec, _bits(x).to(dev), values, meta, sc.to(dev), bi.to(dev))
    got = _unbits(out, T, B, N, C_out)
    rep = compare(got, None, s_ref.numpy(), h_ref.numpy(), 1.0)
    assert rep.ok, str(rep)
    assert float(s_ref.mean()) > 0.01
