"""GPU parity of the strided 3x3 halo-tiled kernel (csrc/tile3s.h) against the CPU oracle.

Spike-bit 3x3 / stride 2 / pad 1 convolutions at T = 4 -- the first conv of every downsampling
residual block (MS-ResNet's conv_bn1, models/msresnet.py:130-141; SEW-ResNet's conv1 with a
downsample, models/sewresnet.py:50-66) -- route to the strided kernel.  The oracle is the
restated reference PyTorch path (oracle.reference_path: F.conv2d with stride 2 + eval BN,
models/neurons.py LIF / IF), pinned against a float64 brute-force direct convolution for
strided cases (tests/test_oracle.py).  Cases: both tile shapes (8x8 and 7x7 output tiles),
the reduction split over two wave sets, ragged outputs (tiles hanging over the image edge),
every epilogue mode (the fast hard-reset LIF / IF, the generic one with soft reset, tau != 2,
a membrane state and the per-step traces), fp16 output, and MS-ResNet-34's four strided
layers at the benchmark's batch of 32.
"""
import numpy as np
import pytest
import torch

from oracle import packing as pk
from oracle import reference_path as ref
from sparsesnn_amd import ops
from tests.test_gpu_fused import run_case

pytestmark = pytest.mark.gpu


@pytest.fixture
def tile_route():
    """Small test shapes would take the split-K small-output kernel under automatic routing."""
    ops.set_fused_kernel("tile")
    yield
    ops.set_fused_kernel("auto")


def _spec(case, **kw):
    T, B, C_in, H, W = case.x_seq.shape
    C_out = case.w.shape[0]
    return ops.ConvSpec(T=T, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=3, KW=3, stride=2, padding=1, **kw)


@pytest.mark.parametrize("shape", ["0", "1"])
@pytest.mark.parametrize("ksp", ["1", "2"])
@pytest.mark.parametrize("B,C_in,C_out,H,W", [(3, 128, 64, 15, 9), (2, 128, 128, 28, 28), (2, 256, 64, 14, 14),
                                              (1, 128, 192, 17, 31)])
def test_strided_route_shapes(dev, monkeypatch, tile_route, shape, ksp, B, C_in, C_out, H, W):
    monkeypatch.setenv("SENGINE_AMD_TILE3S_SHAPE", shape)
    monkeypatch.setenv("SENGINE_AMD_TILE3S_KSP", ksp)
    case = ref.make_layer_case(700 + C_in + H + W, T=4, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=3, stride=2,
                               padding=1, fp16_weights=True, p_spike=0.3)
    plan = ops.fused_plan(_spec(case))
    tr = "8" if shape == "0" else "7"
    assert plan.startswith(f"tile3s<T=4,S=2,TR={tr},TC={tr},GPW=1,KSP={ksp},"), plan
    assert plan.split(">")[0].endswith("out=bits,epi=lif_hard"), plan
    rep, _, r, _ = run_case(dev, case, traces=False, v_th=0.5)
    print(plan, rep, float(r.spikes.mean()))
    assert rep.ok, str(rep)
    assert float(r.spikes.mean()) > 0.01


@pytest.mark.parametrize("neuron,tau,v_reset,traces,state", [
    ("if", 2.0, 0.0, False, False),    # fast IF
    ("lif", 3.0, 0.0, False, False),   # generic: tau != 2
    ("lif", 2.0, None, False, False),  # generic: soft reset
    ("lif", 2.0, 0.0, True, False),    # generic: traces (BN output and charged membrane checked)
    ("lif", 2.0, 0.0, False, True),    # generic: membrane state in and out
    ("if", 1.0, 0.3, True, True),
])
def test_strided_neurons(dev, tile_route, neuron, tau, v_reset, traces, state):
    case = ref.make_layer_case(731, T=4, B=2, C_in=64, C_out=128, H=20, W=18, k=3, stride=2, padding=1,
                               fp16_weights=True, p_spike=0.3)
    spec = _spec(case, neuron=neuron, tau=tau, hard_reset=v_reset is not None, v_threshold=0.5,
                 v_reset=v_reset if v_reset is not None else 0.0)
    plan = ops.fused_plan(spec, traces=traces, state=state)
    assert plan.startswith("tile3s<"), plan
    v0 = None
    if state:
        v0 = torch.rand((2, 128, 10, 9), generator=torch.Generator().manual_seed(3)) * 0.4
    rep, x_err, r, v_fin = run_case(dev, case, neuron=neuron, tau=tau, v_reset=v_reset, v_th=0.5, v0=v0,
                                    traces=traces)
    print(plan, rep, x_err, float(r.spikes.mean()))
    assert rep.ok, str(rep)
    assert x_err is None or x_err < 1e-4
    if state:
        assert torch.allclose(v_fin, r.v_final, rtol=1e-3, atol=1e-3)


def test_strided_f16_out(dev, tile_route):
    case = ref.make_layer_case(741, T=4, B=2, C_in=64, C_out=64, H=16, W=16, k=3, stride=2, padding=1,
                               fp16_weights=True, p_spike=0.3)
    plan = ops.fused_plan(_spec(case, out_enc=ops.ENC_F16))
    assert plan.startswith("tile3s<T=4,S=2,TR=8,TC=8,GPW=1,KSP=1,") and "out=f16" in plan, plan
    rep, _, _, _ = run_case(dev, case, out_enc=ops.ENC_F16, traces=False, v_th=0.5)
    assert rep.ok, str(rep)


def test_strided_route_off_matches(dev, monkeypatch, tile_route):
    """SENGINE_AMD_TILE3S=0 hands the same layer back to the LDS-staged kernel: identical spikes."""
    case = ref.make_layer_case(751, T=4, B=2, C_in=128, C_out=128, H=14, W=14, k=3, stride=2, padding=1,
                               fp16_weights=True, p_spike=0.3)
    spec = _spec(case, v_threshold=0.5)
    values, meta, _ = ops.compress_2_4(spec, case.w.to(dev))
    scale, bias = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
    sc, bi = torch.from_numpy(scale).to(dev), torch.from_numpy(bias).to(dev)
    data = torch.from_numpy(pk.seq_to_nhwc_bits(case.x_seq.numpy()).view(np.int32)).to(dev)
    a = ops.fused_sparse_conv_bn_lif(spec, data, values, meta, sc, bi)
    monkeypatch.setenv("SENGINE_AMD_TILE3S", "0")
    assert ops.fused_plan(spec).startswith("lds<")
    b = ops.fused_sparse_conv_bn_lif(spec, data, values, meta, sc, bi)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


# MS-ResNet-34's strided conv_bn1 layers on 224x224 images (stem 7x7/2 -> 112x112), T = 4, batch 32
MS34_STRIDED = [(64, 64, 112), (64, 128, 56), (128, 256, 28), (256, 512, 14)]


@pytest.mark.parametrize("C_in,C_out,H", MS34_STRIDED)
def test_msresnet34_strided_layers_full_size(dev, C_in, C_out, H):
    case = ref.make_layer_case(760 + C_in, T=4, B=32, C_in=C_in, C_out=C_out, H=H, W=H, k=3, stride=2, padding=1,
                               fp16_weights=True, p_spike=0.15)
    plan = ops.fused_plan(_spec(case))
    print(f"{C_in}->{C_out} {H}x{H}/2: {plan}", flush=True)
    assert plan.startswith("tile3s<T=4,S=2,"), plan
    rep, _, r, _ = run_case(dev, case, traces=False, v_th=0.5)
    print(" ", rep, f"rate {float(r.spikes.mean()):.4f}", flush=True)
    assert rep.ok, str(rep)
