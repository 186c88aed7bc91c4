"""GPU: MS-ResNet through the generic graph engine (front end -> passes -> compile_all ->
CUDAGraphEngine), bit-identical to the hand-wired MSResNetEngine, whose every block is
teacher-forced against the oracle in tests/test_gpu_msresnet_net.py.  Small images at depth
18 and 34 with the MS neuron and LIF, and BASELINE config 3 (MS-ResNet-34, 3x224x224, T=4,
batch 32, LIF tau 2 / V_th 1) with graph replays."""
import pytest
import torch

from sparsesnn_amd import frontend, passes
from sparsesnn_amd.compiler import SparseKernelCompiler
from sparsesnn_amd.ms_resnet import MSResNetEngine, random_params
from sparsesnn_amd.runtime import CUDAGraphEngine

pytestmark = pytest.mark.gpu


def build_generic(p, B, depth, neuron, hw, dev):
    ir = frontend.ms_resnet_ir(p, T=4, batch=B, in_hw=hw, depth=depth, neuron=neuron)
    passes.optimize_ir(ir)
    kernels = SparseKernelCompiler(ir, batch_size=B).compile_all()
    return CUDAGraphEngine().build(ir, kernels, T=4, batch_size=B, device=dev)


@pytest.mark.parametrize("depth,neuron,B,hw", [(18, "ms", 2, (64, 64)), (34, "ms", 2, (64, 48)),
                                               (18, "lif", 3, (40, 40)), (34, "lif", 32, (224, 224))])
def test_generic_engine_runs_ms_resnet(dev, depth, neuron, B, hw):
    p = random_params(70 + depth, depth, 1000 if hw[0] == 224 else 10)
    x = torch.randn((B, 3) + hw, generator=torch.Generator().manual_seed(71))
    eng = build_generic(p, B, depth, neuron, hw, dev)
    ref_eng = MSResNetEngine(p, batch=B, T=4, depth=depth, neuron=neuron, in_hw=hw, device=dev)
    assert eng.n_launches == ref_eng.launches, (eng.n_launches, ref_eng.launches)
    assert len(eng.launch_names()) == eng.n_launches
    want = ref_eng.forward(x.to(dev)).clone()
    eager = eng(x.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(eager, want), float((eager - want).abs().max())
    # the last block's real-valued output and sn_out spikes, not only the logits
    last, last_sc = ref_eng.blocks[-1], eng.launches[-2]
    assert last_sc.kind == "fused_sc"
    assert torch.equal(eng._real(last_sc.real_output).reshape(-1), last.y.reshape(-1))
    assert torch.equal(eng._bits(last_sc.output).reshape(-1), last.spk.reshape(-1))
    eng.capture_graph()
    for i in range(3):
        y = eng(x.to(dev))
        torch.cuda.synchronize()
        assert torch.equal(y, want), f"replay {i}"
        _ = (torch.ones(1000, device=dev) * i).sum().item()
