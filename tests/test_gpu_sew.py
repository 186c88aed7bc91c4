"""GPU parity of the SEW-ResNet-18 path: stem, repeated-input neuron,
spike max-pool, fused Conv+BN+LIF+ADD with bit-plane integer activations, head, and the
whole network replayed from a hipGraph, each against the CPU oracle."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import packing as pk
from oracle import reference_path as ref
from oracle import sew_resnet as sr
from sparsesnn_amd import ops
from sparsesnn_amd.sew_resnet import SEWResNet18Engine
from sparsesnn_amd.sparsity import expand_planes
from tests.parity import compare

pytestmark = pytest.mark.gpu


def _bits_to_seq(t: torch.Tensor, T, B, C, H, W, planes=1):
    w = t.cpu().numpy().view(np.uint32).reshape(-1, planes * C // 32)
    if planes == 1:
        return pk.nhwc_bits_to_seq(w, T, B, C, H, W)
    return pk.planes_to_seq(w, planes, T, B, C, H, W)


@pytest.mark.parametrize("layout", [ops.WLAYOUT_OIHW, ops.WLAYOUT_HWIO])
def test_stem_conv_bn_matches_fp32_conv(dev, layout):
    p = sr.make_params(1, bn_random=True)
    x = sr.make_images(2, 3)
    spec = ops.ConvSpec(T=1, B=3, C_in=3, H=32, W=32, C_out=64, KH=7, KW=7, stride=2, padding=3)
    sc, bi = ref.fold_batchnorm(p["bn1.weight"], p["bn1.bias"], p["bn1.running_mean"], p["bn1.running_var"])
    w = p["conv1.weight"] if layout == ops.WLAYOUT_OIHW else p["conv1.weight"].permute(2, 3, 1, 0).contiguous()
    out = ops.stem_conv_bn(spec, x.to(dev), w.to(dev), torch.from_numpy(sc).to(dev), torch.from_numpy(bi).to(dev),
                           layout=layout)
    exp = F.conv2d(x, p["conv1.weight"], None, 2, 3) * torch.from_numpy(sc)[:, None, None] + \
        torch.from_numpy(bi)[:, None, None]
    got = out.cpu().permute(0, 3, 1, 2)
    assert torch.allclose(got, exp, rtol=1e-5, atol=1e-5), float((got - exp).abs().max())


@pytest.mark.parametrize("B,C,H,W,F,K,S,P", [
    (2, 3, 224, 224, 64, 7, 2, 3),   # ImageNet 7x7/2 stem (MS-ResNet, SEW-ResNet at 224)
    (1, 3, 224, 224, 48, 3, 1, 1),   # Spikformer SPS proj_conv: 3x3/1, three 16-channel groups
    (2, 2, 40, 300, 32, 5, 1, 2),    # padded row wider than 256: two column passes of the staging
    (3, 4, 17, 23, 16, 3, 2, 0),     # odd sizes, no padding
    (1, 1, 9, 9, 16, 1, 1, 0),       # 1x1 taps, runtime-KW variant
])
def test_stem_conv_bn_shapes(dev, B, C, H, W, F, K, S, P):
    """The LDS stem kernel (HWIO weights) over stem shapes of the three networks and
    edge geometries, against an fp32 conv + folded BN on the CPU."""
    g = torch.Generator().manual_seed(B * 1000 + C * 100 + K)
    x = torch.randn(B, C, H, W, generator=g)
    w = torch.randn(F, C, K, K, generator=g) / (C * K * K) ** 0.5
    sc = torch.rand(F, generator=g) + 0.5
    bi = torch.randn(F, generator=g) * 0.1
    spec = ops.ConvSpec(T=1, B=B, C_in=C, H=H, W=W, C_out=F, KH=K, KW=K, stride=S, padding=P)
    out = ops.stem_conv_bn(spec, x.to(dev), w.permute(2, 3, 1, 0).contiguous().to(dev), sc.to(dev), bi.to(dev),
                           layout=ops.WLAYOUT_HWIO)
    exp = F_conv(x, w, S, P) * sc[:, None, None] + bi[:, None, None]
    got = out.cpu().permute(0, 3, 1, 2)
    assert got.shape == exp.shape
    assert torch.allclose(got, exp, rtol=1e-5, atol=2e-5), float((got - exp).abs().max())


@pytest.mark.parametrize("shift", [4, 2])
def test_stem_weight_alignment(dev, shift):
    """HWIO weights at a 16-byte (shift 4 floats) or 8-byte (shift 2) offset: the scalar-load
    kernel takes the first, the per-output kernel the second; both match the conv.  The
    fused entries need 16-byte aligned weights and say so."""
    import dataclasses
    g = torch.Generator().manual_seed(shift)
    B, C, H, F_, K = 2, 3, 32, 64, 7
    x = torch.randn(B, C, H, H, generator=g)
    w = torch.randn(F_, C, K, K, generator=g) / (C * K * K) ** 0.5
    sc = torch.rand(F_, generator=g) + 0.5
    bi = torch.randn(F_, generator=g) * 0.1
    n = K * K * C * F_
    buf = torch.zeros(n + shift, device=dev)
    buf[shift:] = w.permute(2, 3, 1, 0).reshape(-1).to(dev)
    wv = buf[shift:]
    spec = ops.ConvSpec(T=1, B=B, C_in=C, H=H, W=H, C_out=F_, KH=K, KW=K, stride=2, padding=3)
    out = ops.stem_conv_bn(spec, x.to(dev), wv, sc.to(dev), bi.to(dev), layout=ops.WLAYOUT_HWIO)
    exp = F_conv(x, w, 2, 3) * sc[:, None, None] + bi[:, None, None]
    assert torch.allclose(out.cpu().permute(0, 3, 1, 2), exp, rtol=1e-5, atol=2e-5)
    nspec = dataclasses.replace(spec, T=4, neuron="lif")
    if shift % 4 == 0:
        _, spk = ops.stem_conv_bn_neuron(nspec, x.to(dev), wv, sc.to(dev), bi.to(dev))
        ref = ops.multistep_neuron_repeat(out.view(-1), 4, "lif", 2.0, 1.0, 0.0)
        torch.cuda.synchronize()
        assert torch.equal(spk.view(-1).cpu(), ref.view(-1).cpu())
    else:
        with pytest.raises(ops.SEngineError):
            ops.stem_conv_bn_neuron(nspec, x.to(dev), wv, sc.to(dev), bi.to(dev))
        with pytest.raises(ops.SEngineError):
            ops.stem_conv_bn_lif_pool(nspec, x.to(dev), wv, sc.to(dev), bi.to(dev))


def F_conv(x, w, stride, padding):
    return F.conv2d(x.double(), w.double(), None, stride, padding).float()


@pytest.mark.parametrize("K,S,P,pk_,ps,pp", [(3, 1, 1, 3, 2, 1), (5, 2, 2, 2, 2, 0)])
def test_stem_lif_pool_fused_runtime_kw(dev, K, S, P, pk_, ps, pp):
    """Fused stem + LIF + max-pool with a tap width other than 7 (runtime-KW variant)
    against the separate entry points: bit-identical spikes and pool."""
    import dataclasses
    B, C, H, W, F_, T = 2, 3, 16, 16, 32, 4
    g = torch.Generator().manual_seed(K * 10 + S)
    x = torch.rand(B, C, H, W, generator=g).to(dev)
    w = (torch.randn(K, K, C, F_, generator=g) * 1.5 / (C * K * K) ** 0.5).to(dev)
    sc = (torch.rand(F_, generator=g) + 0.5).to(dev)
    bi = (torch.randn(F_, generator=g) * 0.3 + 0.5).to(dev)
    spec = ops.ConvSpec(T=1, B=B, C_in=C, H=H, W=W, C_out=F_, KH=K, KW=K, stride=S, padding=P)
    OH = (H + 2 * P - K) // S + 1
    nspec = dataclasses.replace(spec, T=T, neuron="lif", hard_reset=True, tau=2.0, v_threshold=1.0, v_reset=0.0)
    stem = ops.stem_conv_bn(spec, x, w, sc, bi, layout=ops.WLAYOUT_HWIO)
    spk = ops.multistep_neuron_repeat(stem.view(-1), T, "lif", 2.0, 1.0, 0.0)
    pool = ops.maxpool_spikes(spk, T * B, OH, OH, F_, pk_, ps, pp)
    spk_f = torch.empty(T * B, OH, OH, F_ // 32, dtype=torch.int32, device=dev)
    pool_f, _ = ops.stem_conv_bn_lif_pool(nspec, x, w, sc, bi, pk_, ps, pp, spikes=spk_f)
    torch.cuda.synchronize()
    assert torch.equal(spk_f.view(-1).cpu(), spk.view(-1).cpu())
    assert torch.equal(pool_f.view(-1).cpu(), pool.view(-1).cpu())
    assert int(spk.view(torch.int32).ne(0).sum()) > 0


@pytest.mark.parametrize("neuron,v_reset,T,B", [("lif", 0.0, 4, 3), ("if", 0.0, 4, 2), ("lif", None, 2, 2),
                                                ("if", None, 5, 1)])
def test_stem_lif_pool_fused_matches_separate(dev, neuron, v_reset, T, B):
    """One-launch stem + neuron + max-pool against the three separate entry points (the
    separate path is checked against the oracle above): bit-identical spikes and pool."""
    import dataclasses
    p = sr.make_params(3, bn_random=True)
    x = sr.make_images(4, B).to(dev)
    spec = ops.ConvSpec(T=1, B=B, C_in=3, H=32, W=32, C_out=64, KH=7, KW=7, stride=2, padding=3)
    nspec = dataclasses.replace(spec, T=T, neuron=neuron, hard_reset=v_reset is not None, tau=2.0,
                                v_threshold=1.0, v_reset=0.0 if v_reset is None else v_reset)
    sc, bi = ref.fold_batchnorm(p["bn1.weight"], p["bn1.bias"], p["bn1.running_mean"], p["bn1.running_var"])
    sc, bi = torch.from_numpy(sc).to(dev), torch.from_numpy(bi).to(dev)
    w = p["conv1.weight"].permute(2, 3, 1, 0).contiguous().to(dev)
    stem = ops.stem_conv_bn(spec, x, w, sc, bi, layout=ops.WLAYOUT_HWIO)
    spk = ops.multistep_neuron_repeat(stem.view(-1), T, neuron, 2.0, 1.0, v_reset)
    pool = ops.maxpool_spikes(spk, T * B, 16, 16, 64, 3, 2, 1)
    spk_f = torch.empty(T * B, 16, 16, 2, dtype=torch.int32, device=dev)
    pool_f, _ = ops.stem_conv_bn_lif_pool(nspec, x, w, sc, bi, 3, 2, 1, spikes=spk_f)
    torch.cuda.synchronize()
    assert torch.equal(spk_f.view(-1).cpu(), spk.view(-1).cpu())
    assert torch.equal(pool_f.view(-1).cpu(), pool.view(-1).cpu())
    assert int(spk.view(torch.int32).ne(0).sum()) > 0  # the case spikes


@pytest.mark.parametrize("B,H,F,K,S,P,neuron,T,v_reset", [
    (2, 224, 64, 7, 2, 3, "ms", 4, 0.0),    # MS-ResNet-34 stem + first sn1
    (1, 64, 64, 7, 2, 3, "lif", 3, None),   # soft reset, odd T
    (2, 40, 32, 3, 1, 1, "if", 5, 0.0),     # 3x3/1, one 32-channel word
    (2, 56, 32, 3, 2, 1, "lif", 4, 0.0),    # 3x3/2, two 16-channel waves
    (1, 30, 32, 7, 2, 3, "if", 2, None),    # a partial pixel block
])
@pytest.mark.parametrize("mfma", ["0", "1"])
def test_stem_conv_bn_neuron_matches_separate(dev, B, H, F, K, S, P, neuron, T, v_reset, mfma, monkeypatch):
    """One-launch stem + neuron over the repeated output against stem_conv_bn followed by
    multistep_neuron_repeat.  FMA kernel (SENGINE_AMD_STEM_MFMA=0): the fp32 output and the
    spike bits bit-identical.  Matrix-core kernel (3-channel 7x7 / 3x3 stems): its fp32 output
    within fp32 rounding of the FMA kernel's (a different summation order), and its spike bits
    identical to the neuron run over its own output.  Both also with the fp32 output not
    requested."""
    import dataclasses
    monkeypatch.setenv("SENGINE_AMD_STEM_MFMA", mfma)
    g = torch.Generator().manual_seed(H + F + K)
    x = torch.rand(B, 3, H, H, generator=g).to(dev)
    w = (torch.randn(K, K, 3, F, generator=g) * 2.0 / (3 * K * K) ** 0.5).to(dev)
    sc = (torch.rand(F, generator=g) + 0.5).to(dev)
    bi = (torch.randn(F, generator=g) * 0.3).to(dev)
    spec = ops.ConvSpec(T=1, B=B, C_in=3, H=H, W=H, C_out=F, KH=K, KW=K, stride=S, padding=P)
    tau, vth = (0.25, 0.5) if neuron == "ms" else (2.0, 1.0)
    nspec = dataclasses.replace(spec, T=T, neuron=neuron, hard_reset=v_reset is not None, tau=tau, v_threshold=vth,
                                v_reset=0.0 if v_reset is None else v_reset)
    ref_out = ops.stem_conv_bn(spec, x, w, sc, bi, layout=ops.WLAYOUT_HWIO)
    ref_spk = ops.multistep_neuron_repeat(ref_out.view(-1), T, neuron, tau, vth, v_reset)
    out, spk = ops.stem_conv_bn_neuron(nspec, x, w, sc, bi)
    _, spk2 = ops.stem_conv_bn_neuron(nspec, x, w, sc, bi, want_out=False)
    torch.cuda.synchronize()
    if mfma == "1":
        # at most 147 products of |x| < 1 and |w| < ~1: fp32 reordering moves the sum by ~1e-6
        assert torch.allclose(out.cpu(), ref_out.cpu(), rtol=1e-5, atol=1e-4)
        ref_spk = ops.multistep_neuron_repeat(out.view(-1), T, neuron, tau, vth, v_reset)
        torch.cuda.synchronize()
    else:
        assert torch.equal(out.cpu(), ref_out.cpu())
    assert torch.equal(spk.view(-1).cpu(), ref_spk.view(-1).cpu())
    assert torch.equal(spk2.view(-1).cpu(), ref_spk.view(-1).cpu())
    assert int(spk.view(torch.int32).ne(0).sum()) > 0  # the case spikes


def test_stem_lif_pool_rejects_large_images(dev):
    spec = ops.ConvSpec(T=4, B=1, C_in=3, H=64, W=64, C_out=64, KH=7, KW=7, stride=2, padding=3)
    z = torch.zeros(1, 3, 64, 64, device=dev)
    with pytest.raises(ops.SEngineError):
        ops.stem_conv_bn_lif_pool(spec, z, torch.zeros(7, 7, 3, 64, device=dev), torch.ones(64, device=dev),
                                  torch.zeros(64, device=dev))


@pytest.mark.parametrize("neuron,v_reset", [("lif", 0.0), ("if", 0.0), ("lif", None)])
def test_repeat_neuron(dev, neuron, v_reset):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2 * 64 * 9, generator=g) * 1.5 + 0.5
    s = ops.multistep_neuron_repeat(x.to(dev), 4, neuron, 2.0, 1.0, v_reset)
    xs = x[None].repeat(4, 1)
    if neuron == "lif":
        s_ref, h_ref, _ = ref.multistep_lif(xs, 2.0, 1.0, v_reset)
    else:
        s_ref, h_ref, _ = ref.multistep_if(xs, 1.0, v_reset)
    s_gpu = pk.unpack_bits(s.cpu().numpy().view(np.uint32).reshape(-1, 1), 32).reshape(4, -1)
    rep = compare(s_gpu, None, s_ref.numpy(), h_ref.numpy(), 1.0)
    assert rep.ok, str(rep)


@pytest.mark.parametrize("H,W,C", [(16, 16, 64), (7, 9, 32), (1, 1, 64)])
def test_maxpool_spikes(dev, H, W, C):
    rng = np.random.default_rng(H + W)
    s = (rng.random((2, 3, C, H, W)) < 0.2).astype(np.float32)
    bits = torch.from_numpy(pk.seq_to_nhwc_bits(s).view(np.int32)).to(dev)
    out = ops.maxpool_spikes(bits, 6, H, W, C, 3, 2, 1)
    exp = F.max_pool2d(torch.from_numpy(s).flatten(0, 1), 3, 2, 1)
    OH, OW = exp.shape[-2:]
    got = _bits_to_seq(out, 2, 3, C, OH, OW)
    assert np.array_equal(got, exp.view(2, 3, C, OH, OW).numpy())


@pytest.mark.parametrize("planes,HW,C,N_out,T", [
    (2, 1, 64, 10, 4), (1, 4, 64, 10, 4), (3, 2, 96, 37, 4), (2, 1, 512, 100, 4), (1, 49, 512, 1000, 4),
    (3, 9, 2720, 7, 4), (1, 3, 8192, 65, 4),
    # counting-heavy grids (one 1024-thread workgroup per image): Spikformer's token grid,
    # a position stride above HW (T=64, HW=1), a ragged one
    (5, 3136, 384, 1000, 4), (4, 1, 2048, 10, 64), (3, 700, 224, 5, 4)])
def test_sew_head(dev, planes, HW, C, N_out, T):
    rng = np.random.default_rng(planes + HW)
    B = 3
    a = rng.integers(0, 1 << planes, size=(T, B, C, HW, 1))
    bits = torch.from_numpy(pk.seq_to_planes(a, planes).view(np.int32)).to(dev)
    w = torch.randn(N_out, C) * 0.1
    b = torch.randn(N_out) * 0.1
    y = ops.sew_head(bits, T, B, HW, C, planes, w.to(dev), b.to(dev)).cpu()
    feat = torch.from_numpy(a.astype(np.float64)).flatten(3).mean(3).mean(0)
    exp = (feat @ w.T.double() + b.double()).float()
    assert torch.allclose(y, exp, rtol=1e-5, atol=1e-5), float((y - exp).abs().max())


@pytest.mark.parametrize("HW,C,N_out,T,B", [(3136, 384, 1000, 4, 3), (700, 224, 5, 4, 2), (1, 64, 10, 4, 5),
                                             (63, 96, 7, 2, 40)])
def test_sew_head_fp16_stream_split(dev, HW, C, N_out, T, B):
    """The head over an integer-valued fp16 stream (Spikformer's residual stream): counted by one
    workgroup per image (sengine_amd_sew_head) and with the sums split over up to 64 workgroups
    per image through a workspace (sengine_amd_sew_head_ws): identical logits, equal to numpy's
    mean over positions and T followed by the Linear."""
    rng = np.random.default_rng(HW + C)
    a = rng.integers(0, 19, size=(T * B, HW, C))
    x = torch.from_numpy(a).half().to(dev)
    w = torch.randn(N_out, C) * 0.1
    b = torch.randn(N_out) * 0.1
    y1 = ops.sew_head(x, T, B, HW, C, 0, w.to(dev), b.to(dev)).cpu()
    ws = torch.full((B * ops.HEAD_WS_SPLIT * C,), -7, dtype=torch.int32, device=dev)  # stale contents are overwritten
    y2 = ops.sew_head(x, T, B, HW, C, 0, w.to(dev), b.to(dev), workspace=ws).cpu()
    assert torch.equal(y1, y2)
    feat = torch.from_numpy(a.reshape(T, B, HW, C).astype(np.float64)).mean(2).mean(0)
    exp = (feat @ w.T.double() + b.double()).float()
    assert torch.allclose(y2, exp, rtol=1e-5, atol=1e-5), float((y2 - exp).abs().max())
    with pytest.raises(ops.SEngineError):
        ops.sew_head(x, T, B, HW, C, 0, w.to(dev), b.to(dev), workspace=ws[: B * ops.HEAD_WS_SPLIT * C - 1])


@pytest.mark.parametrize("k,stride,in_planes,res_planes,C_in,C_out,H", [(3, 1, 2, 2, 64, 64, 9), (3, 1, 1, 1, 128, 64, 8),
                                                                        (3, 2, 2, 1, 64, 128, 8), (1, 2, 2, 1, 64, 64, 6)])
def test_fused_add_with_bit_plane_inputs(dev, k, stride, in_planes, res_planes, C_in, C_out, H):
    """Conv over an integer (bit-plane) input with plane-expanded weights, plus the fused
    SEW residual add into two output planes, against conv_bn_seq + LIF + add."""
    T, B = 4, 2
    case = ref.make_layer_case(50 + k + in_planes, T=T, B=B, C_in=C_in, C_out=C_out, H=H, W=H, k=k, stride=stride,
                               padding=k // 2, fp16_weights=True, p_spike=0.3)
    rng = np.random.default_rng(7)
    x_int = (case.x_seq.numpy() + (rng.random(case.x_seq.shape) < 0.3) * (in_planes > 1)).astype(np.float32)
    pad = k // 2
    OH = (H + 2 * pad - k) // stride + 1
    res = rng.integers(0, 3 if res_planes == 2 else 2, size=(T, B, C_out, OH, OH))
    spec = ops.ConvSpec(T=T, B=B, C_in=C_in * in_planes, H=H, W=H, C_out=C_out, KH=k, KW=k, stride=stride,
                        padding=pad)
    wx = expand_planes(case.w, in_planes)
    values, meta, _ = ops.compress_2_4(spec, wx.half().to(dev))
    sc, bi = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
    data = torch.from_numpy(pk.seq_to_planes(x_int, in_planes).view(np.int32)).to(dev)
    resd = torch.from_numpy(pk.seq_to_planes(res, res_planes).view(np.int32)).to(dev)
    out = ops.fused_sparse_conv_bn_lif_add(spec, data, values, meta, torch.from_numpy(sc).to(dev),
                                           torch.from_numpy(bi).to(dev), resd, res_planes, 2)
    got = _bits_to_seq(out, T, B, C_out, OH, OH, planes=2)
    r = ref.fused_layer(torch.from_numpy(x_int), case.w, case.bn, stride, pad, 1, "lif", 2.0, 1.0, 0.0)
    spikes_gpu = got - res
    assert set(np.unique(spikes_gpu)) <= {0.0, 1.0}
    rep = compare(spikes_gpu, None, r.spikes.numpy(), r.h.numpy(), 1.0)
    assert rep.ok, str(rep)


@pytest.mark.parametrize("kernel", ["auto", "tile", "direct"])
@pytest.mark.parametrize("res_planes,out_planes,k,H", [(3, 4, 3, 9), (4, 5, 1, 11), (5, 5, 3, 2), (4, 4, 1, 3)])
def test_fused_add_up_to_five_planes(dev, kernel, res_planes, out_planes, k, H):
    """The residual add into 4 and 5 bit planes (integer streams up to 31, Spikformer's
    residual after 8 blocks), every spike-bit kernel family (small outputs take the flat /
    small-M kernels under 'auto'), carries through all planes checked exactly."""
    T, B, C_in, C_out = 4, 2, 128, 64
    case = ref.make_layer_case(90 + res_planes + k + H, T=T, B=B, C_in=C_in, C_out=C_out, H=H, W=H, k=k,
                               padding=k // 2, fp16_weights=True, p_spike=0.3)
    rng = np.random.default_rng(res_planes + H)
    hi = (1 << res_planes) - (1 if out_planes > res_planes else 2)  # spike + residual fits out_planes
    res = rng.integers(0, hi + 1, size=(T, B, C_out, H, H))
    res[0, 0, :, 0, 0] = hi  # the longest carry chain
    spec = ops.ConvSpec(T=T, B=B, C_in=C_in, H=H, W=H, C_out=C_out, KH=k, KW=k, padding=k // 2)
    values, meta, _ = ops.compress_2_4(spec, case.w.half().to(dev))
    sc, bi = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
    data = torch.from_numpy(pk.seq_to_nhwc_bits(case.x_seq.numpy()).view(np.int32)).to(dev)
    resd = torch.from_numpy(pk.seq_to_planes(res, res_planes).view(np.int32)).to(dev)
    ops.set_fused_kernel(kernel)
    try:
        out = ops.fused_sparse_conv_bn_lif_add(spec, data, values, meta, torch.from_numpy(sc).to(dev),
                                               torch.from_numpy(bi).to(dev), resd, res_planes, out_planes)
    finally:
        ops.set_fused_kernel("auto")
    got = _bits_to_seq(out, T, B, C_out, H, H, planes=out_planes)
    r = ref.fused_layer(case.x_seq, case.w, case.bn, 1, k // 2, 1, "lif", 2.0, 1.0, 0.0)
    spikes_gpu = got - res
    assert set(np.unique(spikes_gpu)) <= {0.0, 1.0}
    rep = compare(spikes_gpu, None, r.spikes.numpy(), r.h.numpy(), 1.0)
    assert rep.ok, str(rep)
    assert float(r.spikes.sum()) > 0


@pytest.fixture(scope="module", params=[2, 64])
def sew_case(request):
    """batch 2, and 64: BASELINE config 2's batch, so the blocks run on the kernel instances
    the end-to-end benchmark times (random BN so that every block fires)."""
    B = request.param
    p = sr.make_params(11, bn_random=True, fp16_weights=True)
    x = sr.make_images(12, B)
    rec = {}
    logits = sr.forward(p, x, record=rec)
    return p, x, rec, logits


def test_engine_blocks_teacher_forced(dev, sew_case):
    """Each block on the oracle's own block input: conv1 / downsample spikes and the conv2
    spikes inside the SEW sum, each against the oracle under the parity rule."""
    p, x, rec, _ = sew_case
    T, B = 4, x.shape[0]
    eng = SEWResNet18Engine(p, batch=B, device=dev)
    eng.forward(x.to(dev))
    prev = "maxpool"
    for i, blk in enumerate(eng.blocks):
        xin = rec[prev].numpy()
        xd = torch.from_numpy(pk.seq_to_planes(xin, blk.in_planes).view(np.int32)).to(dev)
        eng.run_block(i, x=xd)
        torch.cuda.synchronize()
        pre = blk.name
        s = blk.stride
        bn1 = sr._bn(p, pre + ".conv1.module.1")
        r1 = ref.fused_layer(torch.from_numpy(xin), p[pre + ".conv1.module.0.weight"], bn1, s, 1, 1, "lif", 2.0, 1.0,
                             0.0)
        s1 = _bits_to_seq(blk.bufs["s1"], T, B, blk.C_out, blk.OH, blk.OW)
        rep1 = compare(s1, None, r1.spikes.numpy(), r1.h.numpy(), 1.0)
        assert rep1.ok, f"{pre}.sn1 {rep1}"
        if blk.downsample is not None:
            bnd = sr._bn(p, pre + ".downsample.0.module.1")
            rd = ref.fused_layer(torch.from_numpy(xin), p[pre + ".downsample.0.module.0.weight"], bnd, s, 0, 1, "lif",
                                 2.0, 1.0, 0.0)
            ident = _bits_to_seq(blk.bufs["ds"], T, B, blk.C_out, blk.OH, blk.OW)
            repd = compare(ident, None, rd.spikes.numpy(), rd.h.numpy(), 1.0)
            assert repd.ok, f"{pre}.downsample {repd}"
        else:
            ident = xin
        bn2 = sr._bn(p, pre + ".conv2.module.1")
        r2 = ref.fused_layer(torch.from_numpy(s1), p[pre + ".conv2.module.0.weight"], bn2, 1, 1, 1, "lif", 2.0, 1.0,
                             0.0)
        out = _bits_to_seq(blk.bufs["out"], T, B, blk.C_out, blk.OH, blk.OW, planes=blk.out_planes)
        s2 = out - ident
        assert set(np.unique(s2)) <= {0.0, 1.0}, pre
        rep2 = compare(s2, None, r2.spikes.numpy(), r2.h.numpy(), 1.0)
        assert rep2.ok, f"{pre}.sn2 {rep2}"
        prev = pre


def test_engine_end_to_end_graph(dev, sew_case):
    """Whole network from one hipGraph replay: stem/max-pool spikes under the parity rule,
    logits against the oracle, and replays identical to the eager run."""
    p, x, rec, logits = sew_case
    B = x.shape[0]
    eng = SEWResNet18Engine(p, batch=B, device=dev)
    eager = eng.forward(x.to(dev)).clone()
    torch.cuda.synchronize()
    stem = _bits_to_seq(eng.stem_spk, 4, B, 64, eng.H1, eng.W1)
    pool = _bits_to_seq(eng.pool_out, 4, B, 64, eng.H2, eng.W2)
    mism_stem = float(np.mean(stem != rec["stem"].numpy()))
    assert mism_stem <= 1e-4, mism_stem
    if mism_stem == 0:
        assert np.array_equal(pool, rec["maxpool"].numpy())
    eng.capture()
    for _ in range(3):
        y = eng.forward(x.to(dev))
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
    err = float((eager.cpu() - logits).abs().max())
    assert err < 5e-2, err  # a near-threshold flip upstream may move a logit by ~1/T of a weight


def test_engine_reference_init_is_silent(dev):
    """With the reference's initialisation (BN identity) the stem never reaches V_th, so the
    logits are the Linear bias -- both in the oracle and on the GPU."""
    p = sr.make_params(5, fp16_weights=True)
    x = sr.make_images(6, 2)
    y_ref = sr.forward(p, x)
    eng = SEWResNet18Engine(p, batch=2, device=dev)
    y = eng.forward(x.to(dev)).cpu()
    assert torch.allclose(y, y_ref, atol=1e-6)
    assert torch.allclose(y, p["fc.bias"].expand_as(y), atol=1e-6)
