"""The two-conv entry (a residual block's conv1 and its downsample on the same input) against
two single fused calls: bit-identical spikes, one launch or two."""
import pytest
import torch

from sparsesnn_amd import ops
from sparsesnn_amd.sparsity import prune_conv_2_4

pytestmark = pytest.mark.gpu


def _conv(dev, g, spec):
    w = prune_conv_2_4(torch.randn(spec.C_out, spec.C_in, spec.KH, spec.KW, generator=g) *
                       (2.0 / (spec.C_in * spec.KH * spec.KW)) ** 0.5).half()
    values, meta, _ = ops.compress_2_4(spec, w.to(dev))
    sc = (torch.rand(spec.C_out, generator=g) + 0.5).to(dev)
    bi = (torch.randn(spec.C_out, generator=g) * 0.2).to(dev)
    return values, meta, sc, bi


@pytest.mark.parametrize("B,C_in,H,C_out,neuron", [
    (64, 64, 8, 128, "lif"),    # SEW-ResNet-18 layer2.0 at batch 64 (small-output kernel)
    (64, 256, 2, 512, "lif"),   # layer4.0: 1x1 output (flat layout)
    (8, 128, 7, 256, "if"),     # ragged position tiles, IF
    (32, 64, 56, 128, "lif"),   # large output: tile / LDS kernels, two launches
    (3, 64, 5, 64, "lif"),      # ragged: 27 positions, a partial 16-position tile
])
def test_pair_matches_two_single_calls(dev, B, C_in, H, C_out, neuron):
    g = torch.Generator().manual_seed(B + C_in + H)
    T = 4
    kw = dict(T=T, B=B, C_in=C_in, H=H, W=H, C_out=C_out, stride=2, neuron=neuron)
    s0 = ops.ConvSpec(KH=3, KW=3, padding=1, **kw)
    s1 = ops.ConvSpec(KH=1, KW=1, padding=0, **kw)
    v0, m0, sc0, bi0 = _conv(dev, g, s0)
    v1, m1, sc1, bi1 = _conv(dev, g, s1)
    n = T * B * H * H * C_in // 32
    rnd = lambda: torch.randint(-2**31, 2**31 - 1, (n,), generator=g, dtype=torch.int32)
    x = (rnd() & rnd()).to(dev)  # spike bits at density ~1/4
    r0 = ops.fused_sparse_conv_bn_lif(s0, x, v0, m0, sc0, bi0)
    r1 = ops.fused_sparse_conv_bn_lif(s1, x, v1, m1, sc1, bi1)
    p0, p1 = ops.fused_sparse_conv_bn_lif_pair(s0, s1, x, v0, m0, sc0, bi0, v1, m1, sc1, bi1)
    torch.cuda.synchronize()
    assert torch.equal(p0.cpu(), r0.cpu())
    assert torch.equal(p1.cpu(), r1.cpu())
    assert int(r0.ne(0).sum()) > 0 and int(r1.ne(0).sum()) > 0


def test_pair_in_a_graph_replays(dev):
    """Captured in a hipGraph and replayed three times with eager work in between."""
    g = torch.Generator().manual_seed(3)
    kw = dict(T=4, B=64, C_in=128, H=4, W=4, C_out=256, stride=2)
    s0 = ops.ConvSpec(KH=3, KW=3, padding=1, **kw)
    s1 = ops.ConvSpec(KH=1, KW=1, padding=0, **kw)
    v0, m0, sc0, bi0 = _conv(dev, g, s0)
    v1, m1, sc1, bi1 = _conv(dev, g, s1)
    x = torch.randint(-2**31, 2**31 - 1, (4 * 64 * 16 * 128 // 32,), generator=g, dtype=torch.int32).to(dev)
    r0 = ops.fused_sparse_conv_bn_lif(s0, x, v0, m0, sc0, bi0)
    r1 = ops.fused_sparse_conv_bn_lif(s1, x, v1, m1, sc1, bi1)
    o0, o1 = torch.zeros_like(r0), torch.zeros_like(r1)
    ops.fused_sparse_conv_bn_lif_pair(s0, s1, x, v0, m0, sc0, bi0, v1, m1, sc1, bi1, out0=o0, out1=o1)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.fused_sparse_conv_bn_lif_pair(s0, s1, x, v0, m0, sc0, bi0, v1, m1, sc1, bi1, out0=o0, out1=o1)
    for _ in range(3):
        o0.zero_()
        o1.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o0.cpu(), r0.cpu()) and torch.equal(o1.cpu(), r1.cpu())


def test_pair_rejects_different_inputs(dev):
    s0 = ops.ConvSpec(T=4, B=2, C_in=64, H=8, W=8, C_out=64, KH=3, KW=3, padding=1)
    s1 = ops.ConvSpec(T=4, B=2, C_in=64, H=4, W=4, C_out=64, KH=1, KW=1, padding=0)
    z = torch.zeros(4 * 2 * 64 * 64 // 32, dtype=torch.int32, device=dev)
    with pytest.raises(ops.SEngineError):
        ops.fused_sparse_conv_bn_lif_pair(s0, s1, z, z, z, z, z, z, z, z, z)
