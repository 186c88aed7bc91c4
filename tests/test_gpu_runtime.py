"""GPU: the generic hipGraph engine (sparsesnn_amd/runtime.py, the reference's CUDAGraphEngine
interface) on a network built from torch modules: 2:4 fused nodes, a dense Conv+BN fallback
node with a standalone IF neuron, planned buffers, eager run and graph replays, against the
oracle's layer chain."""
import numpy as np
import pytest
import torch

from oracle import reference_path as ref
from sparsesnn_amd import passes, sparsity
from sparsesnn_amd.compiler import SparseKernelCompiler
from sparsesnn_amd.ir import EngineIR, KernelVariant
from sparsesnn_amd.runtime import CUDAGraphEngine
from tests.parity import compare, nhwc_seq

pytestmark = pytest.mark.gpu
T, B, H = 4, 2, 16
LAYERS = [  # (C_in, C_out, k, stride, 2:4?, neuron, v_threshold)
    (64, 64, 3, 1, True, "lif", 1.0),
    (64, 128, 3, 2, True, "lif", 1.0),
    (128, 128, 1, 1, False, "if", 1.0),
    (128, 64, 3, 1, True, "lif", 0.5),
]


def _modules(seed=0):
    torch.manual_seed(seed)
    mods = []
    for ci, co, k, s, sparse, neuron, vth in LAYERS:
        conv = torch.nn.Conv2d(ci, co, k, stride=s, padding=k // 2, bias=False)
        with torch.no_grad():
            w = conv.weight * 1.5
            conv.weight.copy_((sparsity.prune_conv_2_4(w) if sparse else w).half().float())
        bn = torch.nn.BatchNorm2d(co).eval()
        with torch.no_grad():
            bn.weight.uniform_(1.0, 3.0)
            bn.bias.normal_(0.3, 0.3)
            bn.running_mean.normal_(0, 0.1)
            bn.running_var.uniform_(0.5, 1.5)
        mods.append((conv, bn, neuron, vth))
    return mods


def _ir(mods):
    ir = EngineIR()
    ir.T = T
    x, shape = "x", (T * B, LAYERS[0][0], H, H)
    for i, (conv, bn, neuron, vth) in enumerate(mods):
        x = passes.add_conv_bn_neuron(ir, f"l{i}", x, shape, conv, bn, neuron, 2.0, vth, 0.0)
        oh = (shape[2] + 2 * (conv.kernel_size[0] // 2) - conv.kernel_size[0]) // conv.stride[0] + 1
        shape = (T * B, conv.out_channels, oh, oh)
    passes.optimize_ir(ir)
    return ir


def _oracle(x, mods):
    for conv, bn, neuron, vth in mods:
        b = ref.BNParams(bn.weight.detach(), bn.bias.detach(), bn.running_mean, bn.running_var, bn.eps)
        k = conv.kernel_size[0]
        r = ref.fused_layer(x, conv.weight.detach(), b, conv.stride[0], k // 2, 1, neuron, 2.0, vth, 0.0)
        x = r.spikes
    return r


def test_engine_runs_the_graph(dev):
    mods = _modules()
    ir = _ir(mods)
    kinds = sorted(n.assigned_kernel.name for n in ir.nodes.values())
    assert kinds.count("FusedSparseConvBNLIF") == 3 and "TileLangConv1x1BN" in kinds and "CUDAVec4IF" in kinds
    kernels = SparseKernelCompiler(ir, batch_size=B).compile_all()
    eng = CUDAGraphEngine().build(ir, kernels, T=T, batch_size=B, device=dev)
    n_tensors = len(eng.tensors)
    assert len(eng.buffers) < n_tensors  # planned reuse
    g = torch.Generator().manual_seed(5)
    x = torch.bernoulli(torch.full((T, B, 64, H, H), 0.3), generator=g)
    eager = eng(x.flatten(0, 1).to(dev))  # NCHW (T*B, C, H, W)
    r = _oracle(x, mods)
    assert float(r.spikes.mean()) > 0.01
    rep = compare(nhwc_seq(eager.float().cpu(), T), None, r.spikes.numpy(), r.h.numpy(), 0.5)
    assert rep.ok, str(rep)
    eng.capture_graph()
    for i in range(3):
        y = eng(x.flatten(0, 1).permute(0, 2, 3, 1).contiguous().to(dev))  # NHWC input
        torch.cuda.synchronize()
        assert torch.equal(y, eager), i
        _ = torch.ones(1000, device=dev).sum()  # eager work between replays
    assert eng.benchmark(warmup=3, n_iters=5) > 0


def test_engine_repeats_static_images_over_T(dev):
    """A (B, C, H, W) input is the same image at every timestep (the reference's
    static-image path, cuda_graph_runtime.py:142-145)."""
    mods = _modules(1)
    ir = _ir(mods)
    eng = CUDAGraphEngine().build(ir, SparseKernelCompiler(ir, batch_size=B).compile_all(), T=T, batch_size=B,
                                  device=dev)
    g = torch.Generator().manual_seed(6)
    img = torch.bernoulli(torch.full((B, 64, H, H), 0.3), generator=g)
    y = eng(img.to(dev))
    r = _oracle(img.unsqueeze(0).repeat(T, 1, 1, 1, 1), mods)
    rep = compare(nhwc_seq(y.float().cpu(), T), None, r.spikes.numpy(), r.h.numpy(), 0.5)
    assert rep.ok, str(rep)
