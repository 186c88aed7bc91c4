"""GPU parity of the direct-staged fp16-input 1x1 kernel (csrc/tile1ds.h) against the CPU oracle.

fp16 NHWC activations (the reference's native call() ABI, sengine/csrc/cpp_executor.cu:909-913,
and the token Linears of a spiking transformer reading the integer residual stream,
models/spikformer.py:103-125) into 1x1 Conv + BN + LIF / IF with 4 or 6 input chunks route to
it.  Cases: 4-wave (256-channel) and 8-wave (512-channel) super-blocks, both reduction lengths,
spike bits and fp16 spikes out, the q / k / v launch's channel-split planes, the reference
call's membrane state, resident workgroups walking many groups (few slots), any fp16 values
(not only 0/1), and the route switched off (the persistent tile1ps kernel then serves the same
layer, same spikes).  The oracle is the restated reference PyTorch path (oracle.reference_path:
F.conv2d + eval BN + models/neurons.py LIF / IF).
"""
import os

import numpy as np
import pytest
import torch

from oracle import packing as pk
from oracle import reference_path as ref
from sparsesnn_amd import ops
from tests.parity import compare, nhwc_seq
from tests.test_gpu_fused import run_case

pytestmark = pytest.mark.gpu


def _spec(C_in, C_out, H, W, B, neuron="lif", out_enc=ops.ENC_BITS):
    return ops.ConvSpec(T=4, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=1, KW=1, stride=1, padding=0, neuron=neuron,
                        in_enc=ops.ENC_F16, out_enc=out_enc)


def _case(seed, C_in, C_out, H, W, B, real=False):
    case = ref.make_layer_case(seed, T=4, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=1, padding=0, fp16_weights=True,
                               p_spike=0.2)
    if real:  # integer-valued fp16 (a residual stream), up to 6
        g = torch.Generator().manual_seed(seed + 1)
        x = torch.randint(0, 7, case.x_seq.shape, generator=g).float() * (torch.rand(case.x_seq.shape, generator=g) < 0.3)
        case = ref.LayerCase(x, case.w * 0.5, case.bn, 1, 0)
    return case


SHAPES = [  # C_in, C_out, H, W, B: (waves per workgroup, chunks)
    (384, 1280, 64, 40, 2),   # 4 waves, 6 chunks: Spikformer's q/k/v launch width
    (384, 1536, 32, 40, 2),   # 8 waves, 6 chunks: fc1
    (256, 1024, 14, 14, 4),   # 8 waves, 4 chunks: the config-1 1x1 layer's shape class
    (256, 768, 16, 24, 2),    # 4 waves, 4 chunks
]


@pytest.mark.parametrize("out_enc", ["bits", "f16"])
@pytest.mark.parametrize("neuron", ["lif", "if"])
@pytest.mark.parametrize("C_in,C_out,H,W,B", SHAPES)
def test_tile1ds_matches_oracle(dev, C_in, C_out, H, W, B, neuron, out_enc):
    oe = ops.ENC_BITS if out_enc == "bits" else ops.ENC_F16
    plan = ops.fused_plan(_spec(C_in, C_out, H, W, B, neuron, oe))
    nw = 8 if C_out % 512 == 0 else 4
    assert plan.startswith(f"tile1ds<T=4,NW={nw},NCH={C_in // 64},in=f16,out={out_enc},"), plan
    print(plan, flush=True)
    case = _case(900 + C_in // 64 + C_out // 64, C_in, C_out, H, W, B)
    kw = dict(neuron="if", v_th=0.5, v_reset=0.0) if neuron == "if" else {}
    rep, _, r, _ = run_case(dev, case, in_enc=ops.ENC_F16, out_enc=oe, traces=False, **kw)
    print(rep, float(r.spikes.mean()))
    assert rep.ok, str(rep)
    assert float(r.spikes.mean()) > 0.002


@pytest.mark.parametrize("slots", ["3", "7"])
@pytest.mark.parametrize("C_in,C_out,H,W,B", [SHAPES[0], SHAPES[1]])
def test_tile1ds_few_workgroups(dev, env, slots, C_in, C_out, H, W, B):
    """Resident workgroups walking hundreds of groups each (the phase ring wraps many times)."""
    env("SENGINE_AMD_PS_SLOTS", int(slots) * (C_out // 512 if C_out % 512 == 0 else C_out // 256))
    case = _case(910 + int(slots), C_in, C_out, H, W, B)
    rep, _, r, _ = run_case(dev, case, in_enc=ops.ENC_F16, traces=False)
    assert rep.ok, str(rep)


@pytest.mark.parametrize("C_in,C_out,H,W,B", [SHAPES[1], SHAPES[2], SHAPES[3]])
def test_tile1ds_state(dev, C_in, C_out, H, W, B):
    """The reference call's form: fp16 in and out with a membrane (V0 read, final V written)."""
    plan = ops.fused_plan(_spec(C_in, C_out, H, W, B, out_enc=ops.ENC_F16), state=True)
    assert plan.startswith("tile1ds<") and plan.split(">")[0].endswith(",state"), plan
    case = _case(920 + C_in // 64, C_in, C_out, H, W, B)
    v0 = torch.rand((B, C_out, H, W), generator=torch.Generator().manual_seed(5)) * 0.6
    rep, _, r, v_fin = run_case(dev, case, in_enc=ops.ENC_F16, out_enc=ops.ENC_F16, traces=False, v0=v0)
    assert rep.ok, str(rep)
    assert torch.allclose(v_fin, r.v_final, rtol=1e-3, atol=1e-3)


def test_tile1ds_integer_stream_input(dev):
    """fp16 integers up to 6 (Spikformer's residual stream), not only 0/1 spikes."""
    C_in, C_out, H, W, B = SHAPES[0]
    case = _case(930, C_in, C_out, H, W, B, real=True)
    rep, _, r, _ = run_case(dev, case, in_enc=ops.ENC_F16, traces=False)
    print(rep, float(r.spikes.mean()))
    assert rep.ok, str(rep)
    assert float(r.spikes.mean()) > 0.002


def test_tile1ds_split_planes(dev):
    """q, k and v as one 1280-channel launch whose spike bits are split into planes of 384
    channels (the fourth plane holds the padding), each plane equal to the oracle's spikes of
    its channels."""
    C_in, C_out, H, W, B, split = 384, 1280, 56, 56, 1, 384
    spec = _spec(C_in, C_out, H, W, B)
    case = _case(940, C_in, C_out, H, W, B)
    OH, OW, M, _ = ops.geometry(spec)
    values, meta, _ = ops.compress_2_4(spec, case.w.to(dev))
    sc, bi = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
    data = case.x_seq.permute(0, 1, 3, 4, 2).reshape(4 * B, H, W, C_in).contiguous().half().to(dev)
    out = ops.fused_sparse_conv_bn_lif_split(spec, data, values, meta, torch.from_numpy(sc).to(dev),
                                             torch.from_numpy(bi).to(dev), split)
    torch.cuda.synchronize()
    r = ref.fused_layer(case.x_seq, case.w, case.bn, 1, 0, 1, "lif", 2.0, 1.0, 0.0)
    for j in range(-(-C_out // split)):
        c0, c1 = j * split, min(C_out, (j + 1) * split)
        bits = out[j].cpu().numpy().view(np.uint32).reshape(-1, split // 32)
        s = torch.from_numpy(pk.unpack_bits(bits, split).reshape(4 * B, OH, OW, split))[..., :c1 - c0]
        rep = compare(nhwc_seq(s, 4), None, r.spikes.numpy()[:, :, c0:c1], r.h.numpy()[:, :, c0:c1], 1.0)
        assert rep.ok, (j, str(rep))


def test_tile1ds_off_matches_tile1ps(dev, env):
    """SENGINE_AMD_TILE1_DS=0 hands the layer back to the persistent tile1ps kernel: identical
    spikes from both kernels."""
    C_in, C_out, H, W, B = SHAPES[0]
    spec = _spec(C_in, C_out, H, W, B)
    case = _case(950, C_in, C_out, H, W, B)
    values, meta, _ = ops.compress_2_4(spec, case.w.to(dev))
    sc, bi = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
    sc_d, bi_d = torch.from_numpy(sc).to(dev), torch.from_numpy(bi).to(dev)
    data = case.x_seq.permute(0, 1, 3, 4, 2).reshape(4 * B, H, W, C_in).contiguous().half().to(dev)
    a = ops.fused_sparse_conv_bn_lif(spec, data, values, meta, sc_d, bi_d)
    env("SENGINE_AMD_TILE1_DS", 0)
    assert ops.fused_plan(spec).startswith("tile1ps<")
    b = ops.fused_sparse_conv_bn_lif(spec, data, values, meta, sc_d, bi_d)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
