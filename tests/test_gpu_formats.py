"""GPU: weight compressor / dense packer / spike (un)packing against the numpy restatement
(byte-identical), the golden config-0 fixture, and the unfused fallback."""
import os

import numpy as np
import pytest
import torch

from oracle import packing as pk
from oracle import reference_path as ref
from sparsesnn_amd import ops
from tests.parity import compare, nhwc_seq

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "cfg0_golden.npz")


@pytest.mark.parametrize("planes", [1, 2])
@pytest.mark.parametrize("shape", [(64, 64, 3, 3), (128, 256, 1, 1), (192, 128, 5, 5)])
def test_compressor_matches_numpy_restatement(dev, planes, shape):
    g = torch.Generator().manual_seed(sum(shape) + planes)
    w = ref.prune_conv_2_4(torch.randn(shape, generator=g) * 0.05)
    if planes == 1:
        w = w.half().float()
    C_out, C_in, KH, KW = shape
    spec = ops.ConvSpec(T=4, B=1, C_in=C_in, H=8, W=8, C_out=C_out, KH=KH, KW=KW, padding=KH // 2,
                        weight_planes=planes)
    for layout, wt in ((ops.WLAYOUT_OIHW, w), (ops.WLAYOUT_HWIO, w.permute(2, 3, 1, 0).contiguous())):
        for dt in (torch.float32, torch.float16):
            if dt == torch.float16 and planes == 2:
                continue
            values, meta, viol = ops.compress_2_4(spec, wt.to(dt).to(dev), layout)
            ev, em, eviol = pk.compress_2_4(w.numpy(), planes)
            assert np.array_equal(values.cpu().numpy().view(np.uint16), ev.reshape(-1))
            assert np.array_equal(meta.cpu().numpy().view(np.uint32), em.reshape(-1))
            assert np.array_equal(viol.cpu().numpy(), eviol)


def test_compressor_reports_violations(dev):
    w = torch.zeros(64, 64, 1, 1)
    w[3, 0:3] = torch.tensor([1.0, 2.0, 3.0]).view(3, 1, 1)
    spec = ops.ConvSpec(T=4, B=1, C_in=64, H=4, W=4, C_out=64, KH=1, KW=1, padding=0)
    with pytest.raises(ops.SEngineError):
        ops.compress_2_4(spec, w.to(dev))
    _, _, viol = ops.compress_2_4(spec, w.to(dev), check_pattern=False)
    assert np.array_equal(viol.cpu().numpy(), pk.compress_2_4(w.numpy())[2])


def test_dense_packer_matches_numpy(dev):
    g = torch.Generator().manual_seed(9)
    w = torch.randn((128, 96, 3, 3), generator=g)
    spec = ops.ConvSpec(T=4, B=1, C_in=96, H=8, W=8, C_out=128, weight_planes=2)
    v = ops.pack_dense_weights(spec, w.to(dev))
    assert np.array_equal(v.cpu().numpy().view(np.uint16), pk.pack_dense(w.numpy(), 2).reshape(-1))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("n_pos,C", [(1, 32), (3, 64), (1000, 96), (4097, 512)])
def test_pack_unpack_roundtrip(dev, dtype, n_pos, C):
    g = torch.Generator().manual_seed(n_pos + C)
    x = (torch.rand((n_pos, C), generator=g) < 0.3).to(dtype)
    bits = ops.pack_spikes(x.to(dev))
    assert np.array_equal(bits.cpu().numpy().view(np.uint32), pk.pack_bits(x.float().numpy()))
    back = ops.unpack_spikes(bits, C, dtype)
    assert torch.equal(back.cpu(), x)


def test_golden_cfg0_fixture(dev):
    """Config 0 against the committed oracle fixture (fp32 weights -> two fp16 planes)."""
    z = np.load(GOLDEN)
    T, B, C, H, W, F, k, s, p = (int(v) for v in z["shape"])
    tau, vth, vr = (float(v) for v in z["lif"])
    spec = ops.ConvSpec(T=T, B=B, C_in=C, H=H, W=W, C_out=F, KH=k, KW=k, stride=s, padding=p, tau=tau,
                        v_threshold=vth, v_reset=vr, weight_planes=2)
    values, meta, _ = ops.compress_2_4(spec, torch.from_numpy(z["w"]).to(dev))
    scale, bias = ref.fold_batchnorm(z["gamma"], z["beta"], z["mean"], z["var"], float(z["eps"]))
    data = torch.from_numpy(z["x_bits"].view(np.int32)).to(dev)
    OH, OW, M, _ = ops.geometry(spec)
    h = torch.empty(T, M, F, device=dev)
    out = ops.fused_sparse_conv_bn_lif(spec, data, values, meta, torch.from_numpy(scale).to(dev),
                                       torch.from_numpy(bias).to(dev), h_trace=h)
    s_gpu = pk.unpack_bits(out.cpu().numpy().view(np.uint32).reshape(-1, F // 32), F)
    s_ref = pk.unpack_bits(z["spikes_bits"], F)
    h_gpu = nhwc_seq(h.view(T * B, OH, OW, F), T)
    rep = compare(nhwc_seq(torch.from_numpy(s_gpu.reshape(T * B, OH, OW, F)), T), h_gpu,
                  nhwc_seq(torch.from_numpy(s_ref.reshape(T * B, OH, OW, F)), T), z["h"], vth)
    print(rep)
    assert rep.ok, str(rep)
    assert rep.spike_mismatch == 0


@pytest.mark.parametrize("in_enc", [ops.ENC_BITS, ops.ENC_F16])
@pytest.mark.parametrize("planes", [1, 2])
def test_dense_fallback_conv_bn_and_neuron(dev, in_enc, planes):
    """Unfused path: dense conv+BN (non-2:4 weights) then the standalone LIF kernel."""
    g = torch.Generator().manual_seed(21)
    T, B, C, H, W, F = 4, 2, 96, 9, 7, 64
    x = torch.bernoulli(torch.full((T, B, C, H, W), 0.2), generator=g)
    w = torch.randn((F, C, 3, 3), generator=g) * (2 / (9 * C)) ** 0.5
    if planes == 1:
        w = w.half().float()
    bn = ref.BNParams(torch.rand(F, generator=g) + 0.5, torch.randn(F, generator=g) * 0.1,
                      torch.randn(F, generator=g) * 0.1, torch.rand(F, generator=g) + 0.5)
    spec = ops.ConvSpec(T=T, B=B, C_in=C, H=H, W=W, C_out=F, in_enc=in_enc, weight_planes=planes)
    blob = ops.pack_dense_weights(spec, w.to(dev))
    scale, bias = ref.fold_batchnorm(bn.gamma, bn.beta, bn.mean, bn.var)
    x_nhwc = x.permute(0, 1, 3, 4, 2).reshape(T * B, H, W, C).contiguous()
    data = (torch.from_numpy(pk.seq_to_nhwc_bits(x.numpy()).view(np.int32)) if in_enc == ops.ENC_BITS
            else x_nhwc.half()).to(dev)
    y = ops.dense_conv_bn(spec, data, blob, torch.from_numpy(scale).to(dev), torch.from_numpy(bias).to(dev))
    r = ref.fused_layer(x, w, bn, 1, 1, 1, "lif", 2.0, 1.0, 0.0)
    assert np.max(np.abs(nhwc_seq(y, T) - r.x.numpy())) < 1e-4
    h = torch.empty(T, y.numel() // T, device=dev)
    spikes = ops.multistep_neuron(y.view(T, -1), T, "lif", 2.0, 1.0, 0.0, out_enc=ops.ENC_F16, h_trace=h)
    rep = compare(nhwc_seq(spikes.view(T * B, H, W, F), T), nhwc_seq(h.view(T * B, H, W, F), T),
                  r.spikes.numpy(), r.h.numpy(), 1.0)
    assert rep.ok, str(rep)


@pytest.mark.parametrize("neuron,tau,v_reset,enc", [("lif", 2.0, 0.0, ops.ENC_BITS), ("if", 2.0, None, ops.ENC_F16),
                                                    ("lif", 3.0, 0.5, ops.ENC_BITS), ("lif", 2.0, None, ops.ENC_F16)])
def test_multistep_neuron_matches_oracle(dev, neuron, tau, v_reset, enc):
    g = torch.Generator().manual_seed(22)
    T, n = 4, 64 * 37
    x = torch.randn((T, n), generator=g) * 1.5
    v0 = torch.rand(n, generator=g)
    state = v0.clone().to(dev)
    h = torch.empty(T, n, device=dev)
    s = ops.multistep_neuron(x.to(dev), T, neuron, tau, 1.0, v_reset, state=state, out_enc=enc, h_trace=h)
    if enc == ops.ENC_BITS:
        s = torch.from_numpy(pk.unpack_bits(s.cpu().numpy().view(np.uint32).reshape(-1, 1), 32).reshape(T, n))
    else:
        s = s.view(T, n)
    if neuron == "lif":
        sr, hr, vr = ref.multistep_lif(x, tau, 1.0, v_reset, v0)
    else:
        sr, hr, vr = ref.multistep_if(x, 1.0, v_reset, v0)
    assert torch.equal(s.float().cpu(), sr)
    assert torch.equal(h.cpu(), hr)  # same fp32 ops in the same order: bit-exact
    assert torch.equal(state.cpu(), vr)
