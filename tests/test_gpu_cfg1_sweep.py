"""Config-1 parity at full size, on the exact launches bench.py times.

the layer sweep 64->64 56x56 k3, 128->128 28x28 k3, 256->256 14x14
k3, 512->512 7x7 k3, 256->1024 14x14 k1 at T=4, batch 32, fp16 2:4 weights, spike density
p in {0.05, 0.15, 0.30}, BN and LIF (tau 2, V_th 1, hard reset, V0 = 0) as config 0.  The
HIP path runs with automatic routing and no traces, i.e. the stateless fast LIF epilogue of
the tile-kernel instances the bench measures (the test asserts the instance by name through
sengine_amd_fused_plan); the oracle is the restated reference PyTorch path
(oracle.reference_path: models/layers.py:26-31 conv + eval BN, models/neurons.py:121-146
LIF).  Per case:
  * spikes of the bench call against the oracle under the acceptance rule of tests/parity.py;
  * a second call with a zeroed state buffer (the same kernel instance, with its state
    epilogue), membrane written back: spikes bit-identical to the first call, final membranes
    within 1e-3 relative of the oracle's wherever the spike history agrees;
  * the same launch at V_th = 0.25, where far more neurons fire (the config's own threshold
    leaves ~0.5 % of outputs spiking), against the oracle on the same conv output;
  * the call exactly as the reference executor issues it (sengine/csrc/cpp_executor.cu:
    704-718,909-913, membranes zeroed first as sengine_reset_membranes does, :1196-1203): the
    exported per-node .so's call(data, weight, state, bn_scale, bn_bias, spikes, stream) with
    fp16 NHWC spikes in, fp16 spikes out, the runtime's fp16 (KH, KW, C_in, C_out) weight and a
    live fp32 (B*OH*OW, C_out) membrane -- its spikes against the oracle and its written-back
    membrane against the oracle's final membrane.
"""
import ctypes
import dataclasses

import numpy as np
import pytest
import torch

from oracle import packing as pk
from oracle import reference_path as ref
from sparsesnn_amd import export, ops
from sparsesnn_amd.compiler import FusedSparseConvBNLIFKernel
from tests.parity import MEMBRANE_RTOL, compare, compare_final, nhwc_seq

pytestmark = pytest.mark.gpu

SHAPES = [(64, 64, 56, 56, 3), (128, 128, 28, 28, 3), (256, 256, 14, 14, 3), (512, 512, 7, 7, 3),
          (256, 1024, 14, 14, 1)]
DENSITIES = (0.05, 0.15, 0.30)
T, B = 4, 32


def _unpack(out, TB, OH, OW, C):
    s = pk.unpack_bits(out.cpu().numpy().view(np.uint32).reshape(-1, C // 32), C)
    return s.reshape(TB, OH, OW, C)


@pytest.fixture(scope="module")
def abi_so(tmp_path_factory):
    """One exported per-node .so per layer shape (the reference's init()/call() ABI)."""
    sos = {}
    d = tmp_path_factory.mktemp("abi")

    def get(spec):
        key = (spec.C_in, spec.C_out, spec.H, spec.W, spec.KH)
        if key not in sos:
            kern = FusedSparseConvBNLIFKernel(spec, "cfg1_%d_%d_%d_%d_%d" % key)
            so = ctypes.CDLL(export.export_kernel_so(kern, str(d / ("kern_%d_%d_%d_%d_%d.so" % key))))
            so.init.restype = ctypes.c_int
            so.call.restype = ctypes.c_int
            so.call.argtypes = [ctypes.c_void_p] * 7
            assert so.init() == 0
            sos[key] = so
        return sos[key]

    yield get
    from sparsesnn_amd import _lib
    torch.cuda.synchronize()
    assert _lib.load().sengine_amd_release_weights() == 0


@pytest.mark.parametrize("p_spike", DENSITIES)
@pytest.mark.parametrize("C_in,C_out,H,W,k", SHAPES)
def test_cfg1_layer_full_size(dev, abi_so, C_in, C_out, H, W, k, p_spike):
    case = ref.make_layer_case(500 + C_in + k + int(100 * p_spike), T=T, B=B, C_in=C_in, C_out=C_out, H=H, W=W,
                               k=k, p_spike=p_spike, fp16_weights=True)
    spec = ops.ConvSpec(T=T, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=k, KW=k, stride=1, padding=k // 2,
                        neuron="lif", tau=2.0, v_threshold=1.0, v_reset=0.0)
    plan = ops.fused_plan(spec)
    print(f"{C_in}->{C_out} {H}x{W} k{k} p{p_spike}: {plan}", flush=True)
    assert plan.startswith(("tile<T=4,", "tile3ps<T=4,", "tile1ps<T=4,")), plan
    assert "epi=lif_hard" in plan and "out=bits" in plan, plan
    plan_st = ops.fused_plan(spec, state=True)  # the same instance, with its state epilogue
    assert plan_st.split(" ")[0].replace(",state", "") == plan.split(" ")[0], (plan, plan_st)
    spec_abi = dataclasses.replace(spec, in_enc=ops.ENC_F16, out_enc=ops.ENC_F16)
    plan_abi = ops.fused_plan(spec_abi, state=True)
    print(f"  reference call(): {plan_abi}", flush=True)
    if k == 1:  # fp16 in and out with a membrane: the direct-staged 1x1 kernel's state form
        assert plan_abi.startswith("tile1ds<T=4,") and "in=f16,out=f16" in plan_abi and ",state>" in plan_abi
    else:
        assert plan_abi.startswith("tile<T=4,KS=3,") and "in=f16,out=f16" in plan_abi

    OH, OW, M, _ = ops.geometry(spec)
    values, meta, _ = ops.compress_2_4(spec, case.w.to(dev))
    scale, bias = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
    scale_d, bias_d = torch.from_numpy(scale).to(dev), torch.from_numpy(bias).to(dev)
    data = torch.from_numpy(pk.seq_to_nhwc_bits(case.x_seq.numpy()).view(np.int32)).to(dev)

    out = ops.fused_sparse_conv_bn_lif(spec, data, values, meta, scale_d, bias_d)
    state = torch.zeros(M, C_out, dtype=torch.float32, device=dev)
    out_st = ops.fused_sparse_conv_bn_lif(spec, data, values, meta, scale_d, bias_d, state=state)
    spec_lo = dataclasses.replace(spec, v_threshold=0.25)
    assert ops.fused_plan(spec_lo).split(" ")[0] == plan.split(" ")[0]
    out_lo = ops.fused_sparse_conv_bn_lif(spec_lo, data, values, meta, scale_d, bias_d)
    torch.cuda.synchronize()

    x = ref.conv_bn_seq(case.x_seq, case.w, case.bn, 1, k // 2)
    s_ref, h_ref, v_ref = ref.multistep_lif(x, 2.0, 1.0, 0.0)
    s_gpu = nhwc_seq(torch.from_numpy(_unpack(out, T * B, OH, OW, C_out)), T)
    rep = compare(s_gpu, None, s_ref.numpy(), h_ref.numpy(), 1.0)
    print("  v_th 1.0 :", rep, f"rate {float(s_ref.mean()):.4f}", flush=True)
    assert rep.ok, str(rep)

    assert torch.equal(out_st, out), "the state-carrying call must fire exactly like the stateless one"
    v_gpu = state.view(B, OH, OW, C_out).permute(0, 3, 1, 2).cpu().numpy()
    rel, n = compare_final(v_gpu, v_ref.numpy(), s_gpu, s_ref.numpy(), 1.0)
    print(f"  final membrane: max rel {rel:.3e} over {n}", flush=True)
    assert n > 0.99 * v_gpu.size and rel <= MEMBRANE_RTOL

    s_ref_lo, h_ref_lo, _ = ref.multistep_lif(x, 2.0, 0.25, 0.0)
    s_gpu_lo = nhwc_seq(torch.from_numpy(_unpack(out_lo, T * B, OH, OW, C_out)), T)
    rep_lo = compare(s_gpu_lo, None, s_ref_lo.numpy(), h_ref_lo.numpy(), 0.25)
    print("  v_th 0.25:", rep_lo, f"rate {float(s_ref_lo.mean()):.4f}", flush=True)
    assert rep_lo.ok, str(rep_lo)
    assert float(s_ref_lo.mean()) > 0.05

    # the reference executor's call: fp16 NHWC in / out, fp16 HWIO weight, live zeroed membrane
    so = abi_so(spec_abi)
    data16 = case.x_seq.permute(0, 1, 3, 4, 2).reshape(T * B, H, W, C_in).contiguous().half().to(dev)
    w_hwio = case.w.permute(2, 3, 1, 0).contiguous().half().to(dev)
    mem = torch.full((M, C_out), 5.0, dtype=torch.float32, device=dev)
    out16 = torch.full((T * B, OH, OW, C_out), 7.0, dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream(dev)
    args = (data16.data_ptr(), w_hwio.data_ptr(), mem.data_ptr(), scale_d.data_ptr(), bias_d.data_ptr(),
            out16.data_ptr(), stream.cuda_stream)
    for _ in range(2):  # the second call starts from the re-zeroed membrane again, like a replay
        mem.zero_()  # sengine_reset_membranes
        assert so.call(*args) == 0
    torch.cuda.synchronize()
    assert bool(((out16 == 0) | (out16 == 1)).all())
    s_abi = nhwc_seq(out16, T)
    rep_abi = compare(s_abi, None, s_ref.numpy(), h_ref.numpy(), 1.0)
    print("  call()   :", rep_abi, flush=True)
    assert rep_abi.ok, str(rep_abi)
    v_abi = mem.view(B, OH, OW, C_out).permute(0, 3, 1, 2).cpu().numpy()
    rel_abi, n_abi = compare_final(v_abi, v_ref.numpy(), s_abi, s_ref.numpy(), 1.0)
    print(f"  call() final membrane: max rel {rel_abi:.3e} over {n_abi}", flush=True)
    assert n_abi > 0.99 * v_abi.size and rel_abi <= MEMBRANE_RTOL
