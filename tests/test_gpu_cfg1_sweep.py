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
  * a second call with a zeroed state buffer (the persistent kernels have no state epilogue, so
    it runs the one-tile or position-major instance of the same shape), membrane written back:
    spikes bit-identical to the first call, final membranes within 1e-3 relative of the
    oracle's wherever the spike history agrees;
  * the same launch at V_th = 0.25, where far more neurons fire (the config's own threshold
    leaves ~0.5 % of outputs spiking), against the oracle on the same conv output.
"""
import dataclasses

import numpy as np
import pytest
import torch

from oracle import packing as pk
from oracle import reference_path as ref
from sparsesnn_amd import ops
from tests.parity import MEMBRANE_RTOL, compare, compare_final, nhwc_seq

pytestmark = pytest.mark.gpu

SHAPES = [(64, 64, 56, 56, 3), (128, 128, 28, 28, 3), (256, 256, 14, 14, 3), (512, 512, 7, 7, 3),
          (256, 1024, 14, 14, 1)]
DENSITIES = (0.05, 0.15, 0.30)
T, B = 4, 32


def _unpack(out, TB, OH, OW, C):
    s = pk.unpack_bits(out.cpu().numpy().view(np.uint32).reshape(-1, C // 32), C)
    return s.reshape(TB, OH, OW, C)


@pytest.mark.parametrize("p_spike", DENSITIES)
@pytest.mark.parametrize("C_in,C_out,H,W,k", SHAPES)
def test_cfg1_layer_full_size(dev, C_in, C_out, H, W, k, p_spike):
    case = ref.make_layer_case(500 + C_in + k + int(100 * p_spike), T=T, B=B, C_in=C_in, C_out=C_out, H=H, W=W,
                               k=k, p_spike=p_spike, fp16_weights=True)
    spec = ops.ConvSpec(T=T, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=k, KW=k, stride=1, padding=k // 2,
                        neuron="lif", tau=2.0, v_threshold=1.0, v_reset=0.0)
    plan = ops.fused_plan(spec)
    print(f"{C_in}->{C_out} {H}x{W} k{k} p{p_spike}: {plan}", flush=True)
    assert plan.startswith(("tile<T=4,", "tile3ps<T=4,", "tile1ps<T=4,")), plan
    assert "epi=lif_hard" in plan and "out=bits" in plan, plan
    plan_st = ops.fused_plan(spec, state=True)
    if plan.startswith("tile<"):
        assert plan_st.split(" ")[0] == plan.split(" ")[0]
    else:  # the persistent kernels have no state epilogue: the state call runs the one-tile kernel
        assert plan_st.startswith("tile1pm<T=4," if k == 1 else "tile<T=4,KS=3,"), plan_st

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
