"""CPU: the MS-ResNet front end (frontend.ms_resnet_ir) and the passes that map it onto the
generic engine's launches (fuse_stem with a kept real output, absorb_membrane_shortcut,
assign_real_convs, fuse_head in the mean-then-pool order), against the structure of
models/msresnet.py:87-161."""
import pytest

from sparsesnn_amd import frontend, passes
from sparsesnn_amd.compiler import RealConvBNKernel, SparseKernelCompiler, StemConvBNKernel
from sparsesnn_amd.ir import KernelVariant, OpType
from sparsesnn_amd.ms_resnet import block_names, random_params
from sparsesnn_amd.runtime import CUDAGraphEngine


@pytest.fixture(scope="module", params=[18, 34])
def ms_ir(request):
    depth = request.param
    p = random_params(5, depth, 10)
    ir = frontend.ms_resnet_ir(p, T=4, batch=2, in_hw=(64, 64), depth=depth, neuron="ms")
    stats = passes.optimize_ir(ir)
    return depth, ir, stats


def _by(ir, kv):
    return [n for n in ir.nodes.values() if n.assigned_kernel == kv]


def test_ms_front_end_inventory(ms_ir):
    depth, ir, stats = ms_ir
    nb = len(block_names(depth))
    nsc = sum(1 for b in block_names(depth) if b[4])
    ops_ = [n.op_type for n in ir.nodes.values()]
    assert ops_.count(OpType.Conv2d) == 1 + 2 * nb + nsc and ops_.count(OpType.BatchNorm) == 0
    assert stats["folded"] == 1 + 2 * nb + nsc
    assert ops_.count(OpType.MS) == 2 * nb + 1 and ops_.count(OpType.Add) == nb and ops_.count(OpType.Tile) == 1
    assert stats["fused"] == nb and stats["shortcuts"] == nb and stats["real_convs"] == nsc
    assert stats["stems"] == 1 and stats["heads"] == 1 and stats["adds"] == 0  # no SEW add here


def test_ms_launches_match_the_hand_wired_engine(ms_ir):
    """stem + (conv_bn1, [shortcut], conv_bn2 + add + next neuron) per block + head: the launch
    count of MSResNetEngine."""
    depth, ir, _ = ms_ir
    eng = CUDAGraphEngine()
    launches, aliases, _ = eng._analyse(ir, ir.topo_order)
    launches = eng._order(launches, aliases, ir.topo_order)
    kinds = [l.kind for l in launches]
    nb = len(block_names(depth))
    nsc = sum(1 for b in block_names(depth) if b[4])
    assert kinds[0] == "stem" and kinds[-1] == "head"
    assert kinds.count("fused") == nb and kinds.count("fused_sc") == nb and kinds.count("real_conv") == nsc
    assert len(kinds) == 1 + 2 * nb + nsc + 1
    stem = next(l for l in launches if l.kind == "stem")
    assert stem.real_output == "conv1.repeat.out"  # kept for block 0's shortcut conv
    first_sc = next(l for l in launches if l.kind == "real_conv")
    assert aliases.get(first_sc.inputs[0], first_sc.inputs[0]) == "conv1.repeat.out"
    for l in launches:
        if l.kind == "fused_sc":  # writes the next neuron's spikes and the real-valued block output
            node = ir.nodes[l.nid]
            assert node.extra_attrs["fusion_slice"] == "Conv2d+Add+MS" and l.real_output.endswith(".add.out")


def test_ms_head_and_specs(ms_ir):
    depth, ir, _ = ms_ir
    head = _by(ir, KernelVariant.CuBLASGemm)[0]
    assert head.extra_attrs["fusion_slice"] == "TemporalMean+GlobalAvgPool+Flatten+Gemm"
    assert head.extra_attrs["head_input"] == "sn_out.out"
    kernels = SparseKernelCompiler(ir, batch_size=2).compile_all()
    by_name = {ir.nodes[nid].name: k for nid, k in kernels.items()}
    stem = by_name["conv1.module.0"]
    assert isinstance(stem, StemConvBNKernel) and stem.spec.neuron == "ms" and stem.spec.tau == 0.25
    assert stem.spec.v_threshold == 0.5 and stem.pool is None
    c2 = by_name["conv2_x.0.conv_bn2.module.0"]
    assert c2.spec.neuron == "ms" and c2.spec.tau == 0.25 and c2.spec.C_out == 64
    sc = by_name["conv2_x.0.shortcut.module.0"]
    assert isinstance(sc, RealConvBNKernel) and sc.spec.stride == 2 and sc.spec.KH == 1
    assert (kernels[head.id].T, kernels[head.id].HW, kernels[head.id].C) == (4, 4, 512)


def test_ms_lif_neuron_option():
    p = random_params(6, 18, 10)
    ir = frontend.ms_resnet_ir(p, T=4, batch=1, in_hw=(32, 32), depth=18, neuron="lif")
    passes.optimize_ir(ir)
    assert {n.op_type for n in ir.nodes.values()} & {OpType.MS} == set()
    kernels = SparseKernelCompiler(ir, batch_size=1).compile_all()
    fused = [k for k in kernels.values() if hasattr(k, "in_planes")]
    assert fused and all(k.spec.neuron == "lif" and k.spec.tau == 2.0 and k.spec.v_threshold == 1.0 for k in fused)
