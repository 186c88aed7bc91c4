"""GPU: SEW-ResNet-18 through the generic path the reference takes --
module tree -> EngineIR (sparsesnn_amd/frontend.py) -> optimize_ir -> compile_all ->
CUDAGraphEngine -> hipGraph (sengine/engine.py:91-191, cuda_graph_runtime.py:28-198) --
against the hand-wired SEWResNet18Engine (same kernels: logits bit-identical) and the
oracle (models/sewresnet.py:190-210 restated)."""
import numpy as np
import pytest
import torch

from oracle import sew_resnet as sr
from sparsesnn_amd import frontend, passes
from sparsesnn_amd.compiler import SparseKernelCompiler
from sparsesnn_amd.runtime import CUDAGraphEngine
from sparsesnn_amd.sew_resnet import SEWResNet18Engine
from tests.sew_modules import SEWResNet18Modules

pytestmark = pytest.mark.gpu


def build_engine(model, B, dev):
    ir = frontend.sew_resnet_ir(model, T=4, batch=B, in_hw=(32, 32))
    passes.optimize_ir(ir)
    kernels = SparseKernelCompiler(ir, batch_size=B).compile_all()
    return CUDAGraphEngine().build(ir, kernels, T=4, batch_size=B, device=dev)


@pytest.mark.parametrize("B,bn_random", [(2, True), (64, True), (64, False)])
def test_generic_engine_runs_sew_resnet18(dev, B, bn_random):
    p = sr.make_params(11, bn_random=bn_random, fp16_weights=True)
    x = sr.make_images(12, B)
    model = SEWResNet18Modules.from_params(p, neuron_type="lif",
                                           neuron_kw=dict(tau=2.0, v_threshold=1.0, v_reset=0.0))
    eng = build_engine(model, B, dev)
    ref_eng = SEWResNet18Engine(p, batch=B, device=dev)
    assert eng.n_launches == ref_eng.launches == 18, (eng.n_launches, ref_eng.launches)
    eager = eng(x.to(dev))
    want = ref_eng.forward(x.to(dev)).clone()
    torch.cuda.synchronize()
    assert torch.equal(eager, want), float((eager - want).abs().max())
    eng.capture_graph()
    for _ in range(3):
        y = eng(x.to(dev))
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
    logits = sr.forward(p, x)
    err = float((eager.cpu() - logits).abs().max())
    assert err < 5e-2, err  # a near-threshold flip upstream may move a logit by ~1/T of a weight
    dens = eng.spike_density()
    assert len(dens) == 1 + 19 and all(0.0 <= v <= 1.0 for v in dens.values())
    if bn_random:
        assert min(dens.values()) > 0.0
    print({k: round(v, 4) for k, v in dens.items()})


def test_generic_engine_block_outputs_match_hand_wired(dev):
    """Every block output (SEW sum planes) of the generic engine equals the hand-wired
    engine's, bit for bit."""
    B = 4
    p = sr.make_params(21, bn_random=True, fp16_weights=True)
    x = sr.make_images(22, B).to(dev)
    eng = build_engine(p, B, dev)
    ref_eng = SEWResNet18Engine(p, batch=B, device=dev)
    eng(x)
    ref_eng.forward(x)
    torch.cuda.synchronize()
    names = {eng.ir.nodes[l.nid].name: l for l in eng.launches}
    for blk in ref_eng.blocks:
        l = names[blk.name + ".conv2.module.0"]
        got = eng._bits(l.output).reshape(-1)
        assert torch.equal(got, blk.bufs["out"].reshape(-1)), blk.name
