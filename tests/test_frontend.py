"""CPU: the SEW-ResNet front end (sparsesnn_amd/frontend.py) and the network-level passes
(sparsesnn_amd/passes.py) on a module tree with the reference's sew_resnet18 structure."""
import numpy as np
import pytest
import torch

from oracle import sew_resnet as sr
from sparsesnn_amd import frontend, passes
from sparsesnn_amd.compiler import SparseKernelCompiler
from sparsesnn_amd.ir import KernelVariant, OpType
from tests.sew_modules import SEWResNet18Modules


@pytest.fixture(scope="module")
def ir_and_params():
    p = sr.make_params(3, num_classes=100, fp16_weights=True)
    model = SEWResNet18Modules.from_params(p, neuron_type="lif",
                                           neuron_kw=dict(tau=2.0, v_threshold=1.0, v_reset=0.0))
    ir = frontend.sew_resnet_ir(model, T=4, batch=2, in_hw=(32, 32))
    stats = passes.optimize_ir(ir)
    return ir, stats, p


def _by_kernel(ir, kv):
    return [n for n in ir.nodes.values() if n.assigned_kernel == kv]


def test_front_end_node_inventory(ir_and_params):
    ir, stats, _ = ir_and_params
    ops_ = [n.op_type for n in ir.nodes.values()]
    assert ops_.count(OpType.Conv2d) == 20 and ops_.count(OpType.Add) == 8
    assert ops_.count(OpType.BatchNorm) == 0 and stats["folded"] == 20  # every BN folded into its conv
    assert ops_.count(OpType.LIF) == 20 and ops_.count(OpType.Tile) == 1
    assert ops_.count(OpType.Gemm) == 1 and ops_.count(OpType.TemporalMean) == 1
    assert stats["fused"] == 19 and stats["sparse"] == 19 and stats["stems"] == 1 and stats["adds"] == 8
    assert stats["heads"] == 1 and stats["pools"] == 0


def test_fusion_slices(ir_and_params):
    ir, _, _ = ir_and_params
    stem = _by_kernel(ir, KernelVariant.TileLangStemConvBN)
    assert len(stem) == 1 and stem[0].extra_attrs["fusion_slice"] == "Conv2d+Tile+LIF+MaxPool"
    fused = _by_kernel(ir, KernelVariant.FusedSparseConvBNLIF)
    with_add = [n for n in fused if n.extra_attrs["fusion_slice"] == "Conv2d+LIF+Add"]
    assert len(with_add) == 8 and all(n.name.endswith("conv2.module.0") for n in with_add)
    for n in with_add:  # the residual is the block input or the downsample's spikes
        res = n.extra_attrs["residual_input"]
        prod = ir.nodes[n.extra_attrs["residual_nid"]]
        assert prod.output_names[0] == res
    head = _by_kernel(ir, KernelVariant.CuBLASGemm)
    assert len(head) == 1 and head[0].extra_attrs["fusion_slice"] == "GlobalAvgPool+Flatten+TemporalMean+Gemm"
    absorbed = set()
    for n in ir.nodes.values():
        absorbed.update(n.extra_attrs.get("absorbed_nids", []))
    for n in ir.nodes.values():  # every non-launching node is absorbed
        if n.assigned_kernel == KernelVariant.ZeroCost:
            assert n.id in absorbed, n.name


def test_activation_planes(ir_and_params):
    """SEW sums: block outputs hold identity + spike, so values reach 3 after two blocks
    without a downsample (2 bit planes); downsample blocks restart from binary identities."""
    ir, _, _ = ir_and_params
    fused = {n.name: n for n in _by_kernel(ir, KernelVariant.FusedSparseConvBNLIF)}
    assert fused["layer1.0.conv1.module.0"].extra_attrs["in_planes"] == 1
    assert fused["layer1.0.conv2.module.0"].extra_attrs["out_planes"] == 2
    assert fused["layer1.1.conv1.module.0"].extra_attrs["in_planes"] == 2
    assert fused["layer1.1.conv2.module.0"].extra_attrs["out_planes"] == 2  # max 3
    assert fused["layer2.0.downsample.0.module.0"].extra_attrs["in_planes"] == 2
    assert fused["layer2.0.conv2.module.0"].extra_attrs["out_planes"] == 2  # binary identity + spike
    head = _by_kernel(ir, KernelVariant.CuBLASGemm)[0]
    assert head.extra_attrs["in_planes"] == 2


def test_state_dict_and_module_tree_agree(ir_and_params):
    ir, _, p = ir_and_params
    ir2 = frontend.sew_resnet_ir(p, T=4, batch=2, in_hw=(32, 32))
    passes.optimize_ir(ir2)
    assert [n.name for n in ir.nodes.values()] == [n.name for n in ir2.nodes.values()]
    for n, n2 in zip(ir.nodes.values(), ir2.nodes.values()):
        assert n.assigned_kernel == n2.assigned_kernel and n.extra_attrs == n2.extra_attrs
        if n.bn_scale is not None:
            assert np.array_equal(n.bn_scale, n2.bn_scale) and np.array_equal(n.bn_bias, n2.bn_bias)


def test_compiler_specs(ir_and_params):
    """Kernel objects: plane-expanded reductions for integer inputs, the stem and the head."""
    ir, _, _ = ir_and_params
    kernels = SparseKernelCompiler(ir, batch_size=2).compile_all()
    by_name = {ir.nodes[nid].name: k for nid, k in kernels.items()}
    k = by_name["layer1.1.conv1.module.0"]
    assert k.spec.C_in == 128 and k.in_planes == 2
    stem = by_name["conv1"]
    assert stem.pool == (3, 2, 1) and stem.spec.B == 2 and stem.spec.T == 4 and stem.spec.KH == 7
    head = by_name["fc"]
    assert (head.T, head.B, head.HW, head.C, head.planes) == (4, 2, 1, 512, 2)


def test_unabsorbed_add_is_rejected_by_the_runtime():
    from sparsesnn_amd.ir import EngineIR, Node
    from sparsesnn_amd.ops import SEngineError
    from sparsesnn_amd.runtime import CUDAGraphEngine
    ir = EngineIR()
    ir.add_node(Node(0, "add", OpType.Add, input_names=["a", "b"], output_names=["c"],
                     input_shapes=[(4, 64, 2, 2)], output_shapes=[(4, 64, 2, 2)]))
    with pytest.raises(SEngineError, match="not absorbed"):
        CUDAGraphEngine()._analyse(ir, ir.topo_order)


def test_non_add_connection_rejected():
    p = sr.make_params(3, num_classes=10)
    m = SEWResNet18Modules.from_params(p)
    m.connect_f = "IAND"
    with pytest.raises(ValueError, match="ADD"):
        frontend.sew_resnet_ir(m, T=4, batch=1)


@pytest.mark.parametrize("neuron_type,kw,want", [
    ("if", {}, ("IF", 1.0, 1.0, 0.0, True)),  # the reference default (models/sewresnet.py:124)
    ("if", dict(v_threshold=0.75, v_reset=None), ("IF", 1.0, 0.75, 0.0, False)),
    ("lif", dict(tau=3.0, v_threshold=0.5, v_reset=0.25), ("LIF", 3.0, 0.5, 0.25, True)),
])
def test_neuron_settings_from_the_nested_neuron(neuron_type, kw, want):
    """The kind comes from the model's neuron_type and the settings from the multi-step
    wrapper's single-step `neuron` member, as in the reference's module tree; the function's
    own defaults (LIF, tau 2) must not leak into a model that says otherwise."""
    p = sr.make_params(3, num_classes=10)
    m = SEWResNet18Modules.from_params(p, neuron_type=neuron_type, neuron_kw=kw)
    assert not hasattr(m.sn1, "tau") and not hasattr(m.sn1, "v_threshold")  # nested like the reference
    ir = frontend.sew_resnet_ir(m, T=4, batch=1)
    neurons = [n for n in ir.nodes.values() if n.op_type in (OpType.LIF, OpType.IF)]
    assert len(neurons) == 20
    kind, tau, vth, vreset, hard = want
    for n in neurons:
        assert n.op_type.name == kind
        np_ = n.neuron_params
        assert (np_.tau, np_.v_threshold, np_.v_reset, np_.hard_reset) == (tau, vth, vreset, hard), n.name
    # the compiled kernel objects carry the same neuron
    passes.optimize_ir(ir)
    kernels = SparseKernelCompiler(ir, batch_size=1).compile_all()
    fused = [k for k in kernels.values() if hasattr(k, "in_planes")]
    assert fused and all(k.spec.neuron == kind.lower() and k.spec.v_threshold == vth for k in fused)
    assert all(k.spec.tau == (tau if kind == "LIF" else 2.0) and k.spec.hard_reset == hard for k in fused)


def test_neuron_class_names_without_neuron_type():
    """A tree without neuron_type: the kind follows the first neuron's class."""
    p = sr.make_params(3, num_classes=10)
    m = SEWResNet18Modules.from_params(p, neuron_type="lif", neuron_kw=dict(tau=4.0))
    del m.neuron_type
    ir = frontend.sew_resnet_ir(m, T=4, batch=1, neuron="if")
    n = next(n for n in ir.nodes.values() if n.name == "sn1")
    assert n.op_type == OpType.LIF and n.neuron_params.tau == 4.0
