"""GPU parity of the MS-ResNet pieces: the MSNeuron as a neuron kind of
every fused kernel and of the unfused neuron kernel, and the membrane-shortcut epilogue
(y = BN(conv) + residual stored as fp32, the neuron fired on y), against the oracle."""
import numpy as np
import pytest
import torch

from oracle import packing as pk
from oracle import reference_path as ref
from sparsesnn_amd import ops
from tests.parity import compare, nhwc_seq
from tests.test_gpu_fused import run_case

pytestmark = pytest.mark.gpu

DECAY, THRESH = 0.25, 0.5  # models/msresnet.py:20-21


@pytest.mark.parametrize("kernel", ["auto", "lds", "direct", "tile"])
@pytest.mark.parametrize("k,stride,H,C_in,C_out", [(3, 1, 12, 64, 64), (3, 2, 11, 128, 64), (1, 1, 9, 256, 128),
                                                   (3, 1, 2, 128, 128)])
def test_ms_neuron_in_fused_kernels(dev, kernel, k, stride, H, C_in, C_out):
    """Conv + BN + MSNeuron (hard reset through the carried (1 - spike) factor)."""
    ops.set_fused_kernel(kernel)
    try:
        case = ref.make_layer_case(80 + k + stride + H, T=4, B=2, C_in=C_in, C_out=C_out, H=H, W=H, k=k,
                                   stride=stride, padding=k // 2, fp16_weights=True, p_spike=0.25)
        rep, x_err, r, _ = run_case(dev, case, neuron="ms", tau=DECAY, v_th=THRESH, v_reset=0.0)
        print(rep, x_err, float(r.spikes.mean()))
        assert rep.ok, str(rep)
        assert float(r.spikes.mean()) > 0.01
    finally:
        ops.set_fused_kernel("auto")


@pytest.mark.parametrize("decay", [0.25, 0.3])
def test_ms_neuron_unfused(dev, decay):
    g = torch.Generator().manual_seed(3)
    T, n = 4, 4096
    x = torch.randn(T, n, generator=g) * 0.4 + 0.2
    h_gpu = torch.empty(T, n, device=dev)
    s_gpu = ops.multistep_neuron(x.to(dev), T, "ms", decay, THRESH, 0.0, out_enc=ops.ENC_F16, h_trace=h_gpu)
    s_ref, h_ref, _ = ref.ms_neuron(x, decay, THRESH)
    rep = compare(s_gpu.float().cpu().numpy().reshape(T, n), h_gpu.cpu().numpy().reshape(T, n), s_ref.numpy(),
                  h_ref.numpy(), THRESH)
    assert rep.ok, str(rep)


def _shortcut_case(dev, seed, T, B, C_in, C_out, H, k, stride, neuron, tau, v_th, with_res, with_state,
                   in_planes=1):
    case = ref.make_layer_case(seed, T=T, B=B, C_in=C_in, C_out=C_out, H=H, W=H, k=k, stride=stride,
                               padding=k // 2, fp16_weights=True, p_spike=0.3)
    OH = (H + 2 * (k // 2) - k) // stride + 1
    g = torch.Generator().manual_seed(seed)
    res = torch.randn(T, B, C_out, OH, OH, generator=g) * 0.5 if with_res else None
    v0 = torch.rand(B, C_out, OH, OH, generator=g) * 0.4 if with_state else None
    spec = ops.ConvSpec(T=T, B=B, C_in=C_in, H=H, W=H, C_out=C_out, KH=k, KW=k, stride=stride, padding=k // 2,
                        neuron=neuron, hard_reset=True, tau=tau, v_threshold=v_th, v_reset=0.0)
    values, meta, _ = ops.compress_2_4(spec, case.w.to(dev))
    sc, bi = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
    data = torch.from_numpy(pk.seq_to_nhwc_bits(case.x_seq.numpy()).view(np.int32)).to(dev)
    res_d = None if res is None else res.permute(0, 1, 3, 4, 2).reshape(T * B, OH, OH, C_out).contiguous().to(dev)
    state = None if v0 is None else v0.permute(0, 2, 3, 1).reshape(-1, C_out).contiguous().to(dev)
    y, spk = ops.fused_sparse_conv_bn_add_neuron(spec, data, values, meta, torch.from_numpy(sc).to(dev),
                                                 torch.from_numpy(bi).to(dev), residual=res_d, state=state)
    torch.cuda.synchronize()
    r = ref.shortcut_layer(case.x_seq, case.w, case.bn, res, stride, k // 2, neuron, tau, v_th, 0.0, v0)
    s_gpu = pk.unpack_bits(spk.cpu().numpy().view(np.uint32).reshape(-1, C_out // 32), C_out)
    s_gpu = nhwc_seq(torch.from_numpy(s_gpu.reshape(T * B, OH, OH, C_out)), T)
    y_gpu = nhwc_seq(y, T)
    return s_gpu, y_gpu, r


@pytest.mark.parametrize("kernel", ["auto", "direct", "tile"])
@pytest.mark.parametrize("neuron,tau,v_th", [("ms", DECAY, THRESH), ("lif", 2.0, 1.0), ("ms", 0.3, THRESH)])
@pytest.mark.parametrize("k,stride,H,C_in,C_out", [(3, 1, 10, 64, 64), (3, 2, 9, 64, 128), (1, 1, 7, 128, 64),
                                                   (3, 1, 2, 128, 128)])
def test_membrane_shortcut_epilogue(dev, kernel, neuron, tau, v_th, k, stride, H, C_in, C_out):
    """y = BN(conv) + residual (fp32) and the neuron on y, on every kernel family (3x3 halo
    tile, LDS-staged stride 2, 1x1 tile, flat small output; and the direct kernel)."""
    ops.set_fused_kernel(kernel)
    try:
        s_gpu, y_gpu, r = _shortcut_case(dev, 90 + k + H, 4, 2, C_in, C_out, H, k, stride, neuron, tau, v_th,
                                         True, False)
    finally:
        ops.set_fused_kernel("auto")
    y_ref = r.x.numpy()
    assert np.allclose(y_gpu, y_ref, rtol=1e-4, atol=1e-4), float(np.abs(y_gpu - y_ref).max())
    rep = compare(s_gpu, None, r.spikes.numpy(), r.h.numpy(), v_th)
    assert rep.ok, str(rep)
    assert 0.01 < float(r.spikes.mean()) < 0.99


@pytest.mark.parametrize("with_res,with_state,T", [(False, False, 4), (True, True, 4), (True, False, 2)])
def test_membrane_shortcut_options(dev, with_res, with_state, T):
    s_gpu, y_gpu, r = _shortcut_case(dev, 97, T, 3, 64, 128, 8, 3, 1, "ms", DECAY, THRESH, with_res, with_state)
    assert np.allclose(y_gpu, r.x.numpy(), rtol=1e-4, atol=1e-4)
    rep = compare(s_gpu, None, r.spikes.numpy(), r.h.numpy(), THRESH)
    assert rep.ok, str(rep)


@pytest.mark.parametrize("with_res,with_state", [(True, False), (True, True), (False, False)])
@pytest.mark.parametrize("neuron,tau,v_th", [("ms", DECAY, THRESH), ("lif", 2.0, 1.0)])
@pytest.mark.parametrize("H,W,C_in,C_out,B,shape", [(8, 8, 64, 128, 3, "0"), (13, 11, 128, 64, 2, "0"),
                                                    (14, 8, 64, 64, 2, "1"), (9, 10, 256, 128, 2, "2")])
def test_shortcut_mode_tile(dev, env, with_res, with_state, neuron, tau, v_th, H, W, C_in, C_out, B, shape):
    """The lean membrane-shortcut epilogue of the 3x3 tile kernel (epi=shortcut: next timestep's
    residual rows prefetched, rows moved as whole lines through the cross-row transpose) with
    each tile shape, ragged tiles, with and without residual and membrane state: y, spikes and
    the final membrane against the oracle."""
    env("SENGINE_AMD_TILE_SHAPE", shape)
    ops.set_fused_kernel("tile")
    try:
        T = 4
        spec = ops.ConvSpec(T=T, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=3, KW=3, stride=1, padding=1,
                            neuron=neuron, hard_reset=True, tau=tau, v_threshold=v_th, v_reset=0.0)
        plan = ops.fused_plan(spec, state=with_state, shortcut=True)
        assert "epi=shortcut" in plan and plan.startswith("tile<T=4,KS=3,"), plan
        case = ref.make_layer_case(300 + H + W + C_in // 64, T=T, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=3,
                                   fp16_weights=True, p_spike=0.3)
        g = torch.Generator().manual_seed(H * W)
        res = torch.randn(T, B, C_out, H, W, generator=g) * 0.5 if with_res else None
        v0 = torch.rand(B, C_out, H, W, generator=g) * 0.4 if with_state else None
        values, meta, _ = ops.compress_2_4(spec, case.w.to(dev))
        sc, bi = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
        data = torch.from_numpy(pk.seq_to_nhwc_bits(case.x_seq.numpy()).view(np.int32)).to(dev)
        res_d = None if res is None else res.permute(0, 1, 3, 4, 2).reshape(T * B, H, W, C_out).contiguous().to(dev)
        state = None if v0 is None else v0.permute(0, 2, 3, 1).reshape(-1, C_out).contiguous().to(dev)
        y, spk = ops.fused_sparse_conv_bn_add_neuron(spec, data, values, meta, torch.from_numpy(sc).to(dev),
                                                     torch.from_numpy(bi).to(dev), residual=res_d, state=state)
        torch.cuda.synchronize()
    finally:
        ops.set_fused_kernel("auto")
    r = ref.shortcut_layer(case.x_seq, case.w, case.bn, res, 1, 1, neuron, tau, v_th, 0.0, v0)
    s_gpu = pk.unpack_bits(spk.cpu().numpy().view(np.uint32).reshape(-1, C_out // 32), C_out)
    s_gpu = nhwc_seq(torch.from_numpy(s_gpu.reshape(T * B, H, W, C_out)), T)
    y_gpu = nhwc_seq(y, T)
    assert np.allclose(y_gpu, r.x.numpy(), rtol=1e-4, atol=1e-4), float(np.abs(y_gpu - r.x.numpy()).max())
    rep = compare(s_gpu, None, r.spikes.numpy(), r.h.numpy(), v_th)
    assert rep.ok, str(rep)
    assert 0.01 < float(r.spikes.mean()) < 0.99
    if with_state:
        v_fin = state.view(B, H, W, C_out).permute(0, 3, 1, 2).cpu()
        assert torch.allclose(v_fin, r.v_final, rtol=1e-3, atol=1e-3)
