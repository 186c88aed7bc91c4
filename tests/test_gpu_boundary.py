"""GPU: the three drop-in contracts of the fused node.

1. graph-node contract: torch modules -> EngineIR -> optimize_ir -> FusedSparseConvBNLIF;
2. kernel-object contract: compile_all()[nid](data, weight, state, bn_scale, bn_bias),
   called the way sengine/cuda_graph_runtime.py:616-643 calls it (fp16 NHWC in/out,
   HWIO weight tensor as the runtime allocates it, membrane (B*OH*OW, C_out));
3. native ABI: the exported per-node .so, dlopen'd, init() then call(6 ptrs, stream),
   also captured into a hipGraph and replayed with eager work in between.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import reference_path as ref
from sparsesnn_amd import export, passes, sparsity
from sparsesnn_amd.compiler import SparseKernelCompiler
from sparsesnn_amd.ir import EngineIR, KernelVariant
from tests.parity import compare, nhwc_seq

pytestmark = pytest.mark.gpu
T, B, C, H, W, F = 4, 2, 64, 12, 10, 128


def build(neuron="lif"):
    torch.manual_seed(1)
    conv = torch.nn.Conv2d(C, F, 3, padding=1, bias=False)
    with torch.no_grad():
        conv.weight.copy_(sparsity.prune_conv_2_4(conv.weight * 0.5).half().float())
    bn = torch.nn.BatchNorm2d(F).eval()
    with torch.no_grad():
        bn.weight.uniform_(0.5, 1.5)
        bn.bias.normal_(0, 0.1)
        bn.running_mean.normal_(0, 0.1)
        bn.running_var.uniform_(0.5, 1.5)
    ir = EngineIR()
    ir.T = T
    passes.add_conv_bn_neuron(ir, "blk", "x", (T * B, C, H, W), conv, bn, neuron)
    passes.optimize_ir(ir)
    (cid,) = [n.id for n in ir.nodes.values() if n.assigned_kernel == KernelVariant.FusedSparseConvBNLIF]
    return ir, cid, conv, bn


def inputs(dev, seed=3):
    g = torch.Generator().manual_seed(seed)
    x = torch.bernoulli(torch.full((T, B, C, H, W), 0.25), generator=g)
    return x, x.permute(0, 1, 3, 4, 2).reshape(T * B, H, W, C).contiguous().half().to(dev)


def oracle(x, conv, bn, neuron="lif"):
    b = ref.BNParams(bn.weight.detach(), bn.bias.detach(), bn.running_mean, bn.running_var, bn.eps)
    return ref.fused_layer(x, conv.weight.detach(), b, 1, 1, 1, neuron, 2.0, 1.0, 0.0)


def check(spikes_nhwc, r):
    rep = compare(nhwc_seq(spikes_nhwc, T), None, r.spikes.numpy(), r.h.numpy(), 1.0)
    assert rep.ok, str(rep)


@pytest.mark.parametrize("neuron", ["lif", "if"])
def test_kernel_object_contract(dev, neuron):
    ir, cid, conv, bn = build(neuron)
    node = ir.nodes[cid]
    kern = SparseKernelCompiler(ir, batch_size=B).compile_all()[cid]
    x, data = inputs(dev)
    w_hwio = torch.from_numpy(ir.weights[node.weight_info.name]).permute(2, 3, 1, 0).contiguous().half().to(dev)
    sc = torch.tensor(node.bn_scale, dtype=torch.float32, device=dev)
    bi = torch.tensor(node.bn_bias, dtype=torch.float32, device=dev)
    mem = torch.zeros(B * H * W, F, device=dev)
    spikes = kern(data, w_hwio, mem, sc, bi)
    assert spikes.dtype == torch.float16 and tuple(spikes.shape) == (T * B, H, W, F)
    r = oracle(x, conv, bn, neuron)
    check(spikes.float().cpu(), r)
    # final membrane written back as (B*OH*OW, C_out)
    v = mem.view(B, H, W, F).permute(0, 3, 1, 2).cpu()
    assert torch.allclose(v, r.v_final, atol=1e-4)
    # four-argument form: no membrane
    spikes4 = kern(data, w_hwio, sc, bi)
    assert torch.equal(spikes4.cpu(), spikes.cpu())


def test_exported_so_call_and_graph_replay(dev, tmp_path):
    ir, cid, conv, bn = build()
    node = ir.nodes[cid]
    kern = SparseKernelCompiler(ir, batch_size=B).compile_all()[cid]
    so_path = export.export_all_kernels({cid: kern}, ir, str(tmp_path))[cid]
    so = ctypes.CDLL(so_path)
    so.init.restype = ctypes.c_int
    so.call.restype = ctypes.c_int
    so.call.argtypes = [ctypes.c_void_p] * 7
    assert so.init() == 0
    sw = kern.prepare_weight(torch.from_numpy(ir.weights[node.weight_info.name]).to(dev))
    sc = torch.tensor(node.bn_scale, dtype=torch.float32, device=dev)
    bi = torch.tensor(node.bn_bias, dtype=torch.float32, device=dev)
    x, data = inputs(dev, seed=4)
    mem = torch.zeros(B * H * W, F, device=dev)
    out = torch.empty(T * B, H, W, F, dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream(dev)

    def call():
        return so.call(data.data_ptr(), sw.data_ptr(), mem.data_ptr(), sc.data_ptr(), bi.data_ptr(), out.data_ptr(),
                       stream.cuda_stream)

    assert call() == 0
    torch.cuda.synchronize()
    r = oracle(x, conv, bn)
    check(out.float().cpu(), r)
    eager = out.clone()

    # capture call() into a hipGraph; membranes are zeroed by a fill kernel before each replay
    g = torch.cuda.CUDAGraph()
    mem.zero_()
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        stream_c = torch.cuda.current_stream(dev)
        rc = so.call(data.data_ptr(), sw.data_ptr(), mem.data_ptr(), sc.data_ptr(), bi.data_ptr(), out.data_ptr(),
                     stream_c.cuda_stream)
    assert rc == 0
    for i in range(4):
        out.fill_(7.0)
        mem.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs"
        _ = (torch.ones(1000, device=dev) * i).sum().item()  # eager work between replays
