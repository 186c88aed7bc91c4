"""GPU parity of the gather form of the tile kernel (csrc/tile_kernel.h, KS = 0) against the CPU oracle.

The reference's per-node call() takes fp16 NHWC activations on every conv geometry
(sengine/csrc/cpp_executor.cu:909-913; its im2col gather handles any stride and padding,
sengine/kernels/conv2d_bn_if_t4.py:977-992).  fp16 inputs at T = 4 whose geometry the halo- and
position-tiled forms do not cover (stride-2 3x3 of downsampling blocks, unpadded or dilated 3x3,
5x5, 7x7) run on the gather form: one tap per 64-channel chunk, the tap-shifted fp16 rows staged
into LDS.  Checked against the restated reference PyTorch path (oracle.reference_path, pinned
against a float64 brute-force convolution for stride / padding / dilation in tests/test_oracle.py),
with spike inputs and with arbitrary fp16 values, bit and fp16 outputs, the fast and generic
epilogues, a carried membrane and the per-step traces; and against the direct-gather kernel that
served these layers before.
"""
import numpy as np
import pytest
import torch

from oracle import packing as pk
from oracle import reference_path as ref
from sparsesnn_amd import ops
from tests.parity import compare, nhwc_seq
from tests.test_gpu_fused import run_case

pytestmark = pytest.mark.gpu

GEOMS = [  # (k, stride, pad, dilation, B, C_in, C_out, H, W)
    (3, 2, 1, 1, 2, 128, 64, 15, 13),   # a downsampling block's conv1 (ragged: 8x7 outputs)
    (3, 1, 0, 1, 3, 64, 128, 9, 10),    # unpadded
    (5, 2, 2, 1, 2, 64, 64, 11, 12),
    (7, 2, 3, 1, 1, 64, 64, 16, 16),
    (3, 1, 2, 2, 2, 64, 64, 10, 9),     # dilated
]


def _spec(k, stride, pad, dil, B, C_in, C_out, H, W, **kw):
    return ops.ConvSpec(T=4, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=k, KW=k, stride=stride, padding=pad,
                        dilation=dil, in_enc=ops.ENC_F16, **kw)


def _case(seed, k, stride, pad, dil, B, C_in, C_out, H, W, real=False):
    case = ref.make_layer_case(seed, T=4, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=k, stride=stride, padding=pad,
                               fp16_weights=True, p_spike=0.3)
    if dil != 1 or real:
        x = case.x_seq
        if real:  # any fp16 activation: values in [-2, 2), exact in fp16, half of them zero
            g = torch.Generator().manual_seed(seed + 1)
            v = (torch.rand(x.shape, generator=g) * 4 - 2).half().float()
            x = v * (torch.rand(x.shape, generator=g) < 0.5)
        case = ref.LayerCase(x, case.w, case.bn, stride, pad)
    return case


def _oracle_dil(case, dil, **kw):
    return ref.fused_layer(case.x_seq, case.w, case.bn, case.stride, case.padding, dil, **kw)


@pytest.mark.parametrize("out_enc", [ops.ENC_BITS, ops.ENC_F16])
@pytest.mark.parametrize("k,stride,pad,dil,B,C_in,C_out,H,W", [g for g in GEOMS if g[3] == 1])
def test_gather_matches_oracle(dev, k, stride, pad, dil, B, C_in, C_out, H, W, out_enc):
    spec = _spec(k, stride, pad, dil, B, C_in, C_out, H, W, out_enc=out_enc)
    plan = ops.fused_plan(spec)
    assert plan.startswith(f"tile<T=4,KS=0(gather {k}x{k}/{stride})") and "in=f16" in plan, plan
    case = _case(800 + k + stride + pad, k, stride, pad, dil, B, C_in, C_out, H, W)
    rep, x_err, r, _ = run_case(dev, case, in_enc=ops.ENC_F16, out_enc=out_enc, traces=False, v_th=0.5)
    print(plan, rep, float(r.spikes.mean()))
    assert rep.ok, str(rep)
    # traces (generic epilogue) and a carried membrane (IF)
    rep2, x_err2, _, _ = run_case(dev, case, in_enc=ops.ENC_F16, out_enc=out_enc, traces=True, v_th=0.5)
    assert rep2.ok, str(rep2)
    assert x_err2 < 1e-4
    OH, OW = (H + 2 * pad - k) // stride + 1, (W + 2 * pad - k) // stride + 1
    v0 = torch.rand((B, C_out, OH, OW), generator=torch.Generator().manual_seed(4)) * 0.4
    rep3, _, r3, v_fin = run_case(dev, case, neuron="if", v_th=0.5, v0=v0, in_enc=ops.ENC_F16, out_enc=out_enc,
                                  traces=False)
    assert rep3.ok, str(rep3)
    assert torch.allclose(v_fin, r3.v_final, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("k,stride,pad,dil,B,C_in,C_out,H,W", GEOMS[:2])
def test_gather_real_valued(dev, k, stride, pad, dil, B, C_in, C_out, H, W):
    """Any fp16 activation, not only 0/1 spikes (the ABI's data is fp16)."""
    case = _case(820 + k + stride, k, stride, pad, dil, B, C_in, C_out, H, W, real=True)
    rep, x_err, r, _ = run_case(dev, case, in_enc=ops.ENC_F16, traces=True, v_th=0.5)
    print(rep, x_err, float(r.spikes.mean()))
    assert rep.ok, str(rep)
    assert x_err < 1e-3


def test_gather_dilated(dev):
    """Dilation 2 (run_case builds stride / padding from the case; the dilation goes through the
    spec here): spikes and membranes against the oracle's dilated convolution."""
    k, stride, pad, dil, B, C_in, C_out, H, W = GEOMS[4]
    case = _case(830, k, stride, pad, dil, B, C_in, C_out, H, W)
    spec = _spec(k, stride, pad, dil, B, C_in, C_out, H, W, v_threshold=0.5)
    assert ops.fused_plan(spec).startswith("tile<T=4,KS=0(gather")
    OH, OW, M, _ = ops.geometry(spec)
    values, meta, _ = ops.compress_2_4(spec, case.w.to(dev))
    scale, bias = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
    data = case.x_seq.permute(0, 1, 3, 4, 2).reshape(4 * B, H, W, C_in).contiguous().half().to(dev)
    h_tr = torch.empty(4, M, C_out, dtype=torch.float32, device=dev)
    out = ops.fused_sparse_conv_bn_lif(spec, data, values, meta, torch.from_numpy(scale).to(dev),
                                       torch.from_numpy(bias).to(dev), h_trace=h_tr)
    torch.cuda.synchronize()
    s_gpu = pk.unpack_bits(out.cpu().numpy().view(np.uint32).reshape(-1, C_out // 32), C_out)
    s_gpu = torch.from_numpy(s_gpu.reshape(4 * B, OH, OW, C_out))
    r = _oracle_dil(case, dil, neuron="lif", tau=2.0, v_threshold=0.5, v_reset=0.0)
    rep = compare(nhwc_seq(s_gpu, 4), nhwc_seq(h_tr.view(4 * B, OH, OW, C_out), 4), r.spikes.numpy(), r.h.numpy(),
                  0.5)
    print(rep, float(r.spikes.mean()))
    assert rep.ok, str(rep)


def test_gather_off_matches_direct(dev, monkeypatch):
    """SENGINE_AMD_GATHER=0 hands the layer back to the direct-gather kernel: same spikes."""
    k, stride, pad, dil, B, C_in, C_out, H, W = GEOMS[0]
    case = _case(840, k, stride, pad, dil, B, C_in, C_out, H, W)
    spec = _spec(k, stride, pad, dil, B, C_in, C_out, H, W, v_threshold=0.5)
    values, meta, _ = ops.compress_2_4(spec, case.w.to(dev))
    scale, bias = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
    sc, bi = torch.from_numpy(scale).to(dev), torch.from_numpy(bias).to(dev)
    data = case.x_seq.permute(0, 1, 3, 4, 2).reshape(4 * B, H, W, C_in).contiguous().half().to(dev)
    a = ops.fused_sparse_conv_bn_lif(spec, data, values, meta, sc, bi)
    monkeypatch.setenv("SENGINE_AMD_GATHER", "0")
    assert ops.fused_plan(spec).startswith("direct<")
    b = ops.fused_sparse_conv_bn_lif(spec, data, values, meta, sc, bi)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


# MS-ResNet-34's strided conv_bn1 layers as the reference ABI calls them (fp16 in and out), B = 32
@pytest.mark.parametrize("C_in,C_out,H", [(64, 128, 56), (256, 512, 14)])
def test_gather_msresnet34_strided_full_size(dev, C_in, C_out, H):
    case = _case(850 + C_in, 3, 2, 1, 1, 32, C_in, C_out, H, H)
    spec = _spec(3, 2, 1, 1, 32, C_in, C_out, H, H, out_enc=ops.ENC_F16)
    plan = ops.fused_plan(spec, state=True)
    print(plan, flush=True)
    assert plan.startswith("tile<T=4,KS=0(gather 3x3/2)"), plan
    v0 = torch.zeros((32, C_out, H // 2, H // 2))
    rep, _, r, v_fin = run_case(dev, case, in_enc=ops.ENC_F16, out_enc=ops.ENC_F16, traces=False, v_th=0.5, v0=v0)
    print(rep, float(r.spikes.mean()), flush=True)
    assert rep.ok, str(rep)
    assert torch.allclose(v_fin, r.v_final, rtol=1e-3, atol=1e-3)
