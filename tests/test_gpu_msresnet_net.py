"""GPU parity of MS-ResNet-18/34 as whole networks: the fp32 shortcut
conv, every block teacher-forced on the oracle's own block input, the whole forward from one
hipGraph replay against the oracle's logits, and one image at the config-3 shape (224x224,
depth 34, LIF tau 2 / V_th 1)."""
import numpy as np
import pytest
import torch

from oracle import ms_resnet as ms
from oracle import packing as pk
from oracle import reference_path as ref
from sparsesnn_amd import ops
from sparsesnn_amd.ms_resnet import MSResNetEngine
from tests.parity import compare, nhwc_seq

pytestmark = pytest.mark.gpu

NEURONS = {"ms": (0.25, 0.5), "lif": (2.0, 1.0)}


def _bits_to_seq(bits, T, B, C, H, W):
    a = pk.unpack_bits(bits.cpu().numpy().view(np.uint32).reshape(-1, C // 32), C)
    return np.ascontiguousarray(a.reshape(T, B, H, W, C).transpose(0, 1, 4, 2, 3)).astype(np.float32)


def _to_nhwc(x_seq):
    """(T, B, C, H, W) -> (T*B, H, W, C) contiguous."""
    T, B, C, H, W = x_seq.shape
    return x_seq.permute(0, 1, 3, 4, 2).reshape(T * B, H, W, C).contiguous()


@pytest.mark.parametrize("layout", [ops.WLAYOUT_OIHW, ops.WLAYOUT_HWIO])
@pytest.mark.parametrize("stride,C_in,C_out,H,in_T", [(2, 64, 128, 7, 4), (1, 128, 64, 5, 4), (2, 64, 64, 9, 1),
                                                      (2, 256, 512, 14, 4)])
def test_real_conv_bn_against_oracle(dev, layout, stride, C_in, C_out, H, in_T):
    T, B = 4, 2
    g = torch.Generator().manual_seed(C_in + H + stride)
    x = torch.randn(in_T, B, C_in, H, H, generator=g)
    w = ref.prune_conv_2_4(torch.randn(C_out, C_in, 1, 1, generator=g) * (2.0 / C_in) ** 0.5)
    bn = ref.BNParams(torch.rand(C_out, generator=g) + 0.5, torch.randn(C_out, generator=g) * 0.1,
                      torch.randn(C_out, generator=g) * 0.1, torch.rand(C_out, generator=g) + 0.5)
    sc, bi = ref.fold_batchnorm(bn.gamma, bn.beta, bn.mean, bn.var)
    spec = ops.ConvSpec(T=T, B=B, C_in=C_in, H=H, W=H, C_out=C_out, KH=1, KW=1, stride=stride, padding=0)
    wd = w.to(dev) if layout == ops.WLAYOUT_OIHW else w.reshape(C_out, C_in).t().contiguous().to(dev)
    out = ops.real_conv_bn(spec, _to_nhwc(x).to(dev), wd, torch.from_numpy(sc).to(dev), torch.from_numpy(bi).to(dev),
                           in_T=in_T, layout=layout)
    torch.cuda.synchronize()
    exp = ms.tdbn(x.repeat(T // in_T, 1, 1, 1, 1), w, bn, stride, 0)
    got = torch.from_numpy(nhwc_seq(out, T))
    assert got.shape == exp.shape
    assert torch.allclose(got, exp, rtol=1e-5, atol=1e-5), float((got - exp).abs().max())


@pytest.fixture(scope="module", params=[("ms", 18), ("lif", 34)])
def ms_case(request):
    kind, depth = request.param
    p = ms.make_params(11, depth, num_classes=10, init="lively", fp16_weights=True)
    x = torch.randn(2, 3, 64, 64, generator=torch.Generator().manual_seed(12))
    tau, vth = NEURONS[kind]
    logits, xs = ms.forward(p, x, T=4, depth=depth, kind=kind, tau=tau, v_threshold=vth, keep=True)
    return kind, depth, p, x, logits, xs


def _check_blocks_teacher_forced(dev, eng, p, xs, kind, depth, T, B):
    """Block i of `eng` on the oracle's block input x_i: the sn2 spikes of conv_bn1 under the
    parity rule; the shortcut conv output; and, on the engine's own sn2 spikes, the block
    output y = TDBN2 + shortcut within fp32 rounding and the next neuron's spikes under the
    parity rule.  Returns the per-block spike rates of the oracle."""
    tau, vth = NEURONS[kind]
    rates = []
    for i, (blk, (pre, cin, cout, s, has_sc)) in enumerate(zip(eng.blocks, ms.block_names(depth))):
        xi = xs[i]
        s_in = ms.neuron(xi, kind, tau, vth)
        if i == 0:  # the repeated stem output: one timestep of real input
            x_real, in_T = _to_nhwc(xi[:1]).to(dev), 1
        else:
            x_real, in_T = _to_nhwc(xi).to(dev), T
        x_spk = torch.from_numpy(pk.seq_to_nhwc_bits(s_in.numpy()).view(np.int32)).to(dev)
        eng.run_block(i, x_real=x_real, x_spk=x_spk, in_T=in_T)
        torch.cuda.synchronize()
        r1 = ref.fused_layer(s_in, p[pre + ".conv_bn1.module.0.weight"], ms.bn_of(p, pre + ".conv_bn1.module.1"), s,
                             1, 1, kind, tau, vth, 0.0)
        OH, OW = r1.spikes.shape[-2:]
        s1 = _bits_to_seq(blk.s1, T, B, cout, OH, OW)
        rep1 = compare(s1, None, r1.spikes.numpy(), r1.h.numpy(), vth)
        assert rep1.ok, f"{pre}.sn2 {rep1}"
        if has_sc:
            sc = ms.tdbn(xi, p[pre + ".shortcut.module.0.weight"], ms.bn_of(p, pre + ".shortcut.module.1"), s, 0)
            got_sc = torch.from_numpy(nhwc_seq(blk.sc, T))
            assert torch.allclose(got_sc, sc, rtol=1e-5, atol=1e-5), pre
        else:
            sc = xi
        r2 = ref.shortcut_layer(torch.from_numpy(s1), p[pre + ".conv_bn2.module.0.weight"],
                                ms.bn_of(p, pre + ".conv_bn2.module.1"), sc, 1, 1, kind, tau, vth, 0.0)
        y = nhwc_seq(blk.y, T)
        assert np.allclose(y, r2.x.numpy(), rtol=1e-4, atol=1e-4), (pre, float(np.abs(y - r2.x.numpy()).max()))
        spk = _bits_to_seq(blk.spk, T, B, cout, OH, OW)
        rep2 = compare(spk, None, r2.spikes.numpy(), r2.h.numpy(), vth)
        assert rep2.ok, f"{pre} next neuron {rep2}"
        rates.append(float(r2.spikes.mean()))
    return rates


def test_engine_blocks_teacher_forced(dev, ms_case):
    kind, depth, p, x, _, xs = ms_case
    eng = MSResNetEngine(p, batch=2, T=4, depth=depth, neuron=kind, in_hw=(64, 64), device=dev)
    eng.forward(x.to(dev))
    rates = _check_blocks_teacher_forced(dev, eng, p, xs, kind, depth, 4, 2)
    assert all(0.005 < r < 0.95 for r in rates), rates


def test_engine_end_to_end_graph(dev, ms_case):
    """Whole network: stem spikes under the parity rule, replays of the captured hipGraph
    identical to the eager run, logits against the oracle."""
    kind, depth, p, x, logits, xs = ms_case
    tau, vth = NEURONS[kind]
    eng = MSResNetEngine(p, batch=2, T=4, depth=depth, neuron=kind, in_hw=(64, 64), device=dev)
    eager = eng.forward(x.to(dev)).clone()
    torch.cuda.synchronize()
    stem = _bits_to_seq(eng.stem_spk, 4, 2, 64, eng.H1, eng.W1)
    s_ref = ms.neuron(xs[0], kind, tau, vth).numpy()
    assert float(np.mean(stem != s_ref)) <= 1e-4
    eng.capture()
    for _ in range(3):
        y = eng.forward(x.to(dev))
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
    err = float((eager.cpu() - logits).abs().max())
    assert err < 5e-2, err  # a near-threshold flip upstream moves a logit by ~1/(T*HW) of a weight


@pytest.mark.parametrize("batch", [1, 32])
def test_engine_cfg3_shape(dev, batch):
    """BASELINE config 3's network: MS-ResNet-34, 3x224x224 pixels ~N(0,1), T=4, LIF tau 2 /
    V_th 1, 1000 classes, 2:4 convs, on one image and at the benchmark's batch of 32 (whose
    layers run on the tile-kernel instances the end-to-end figure times).  Every block
    teacher-forced on the oracle's block input (the parity rule is per layer call: over 16
    blocks the real-valued shortcut stream carries any allowed near-threshold flip forward,
    so whole-network spikes drift apart); the captured graph's replays equal the eager
    forward."""
    p = ms.make_params(21, 34, num_classes=1000, init="lively", fp16_weights=True)
    x = torch.randn(batch, 3, 224, 224, generator=torch.Generator().manual_seed(22))
    logits, xs = ms.forward(p, x, T=4, depth=34, kind="lif", tau=2.0, v_threshold=1.0, keep=True)
    eng = MSResNetEngine(p, batch=batch, T=4, depth=34, neuron="lif", in_hw=(224, 224), device=dev)
    assert eng.launches == 1 + 16 * 2 + 4 + 1
    eager = eng.forward(x.to(dev)).clone()
    eng.capture()
    y = eng.forward(x.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(y, eager)
    err = float((y.cpu() - logits).abs().max())
    print(f"end-to-end logits max |diff| {err:.3e} (scale {float(logits.abs().max()):.3e})")
    rates = _check_blocks_teacher_forced(dev, eng, p, xs, "lif", 34, 4, batch)
    assert all(0.005 < r < 0.95 for r in rates), rates
