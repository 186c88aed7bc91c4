"""Graph passes that select the fused 2:4 operator (the hot-path part of sengine/optimizer.py
and sengine/fusion_strategy.py), plus a small front end that builds Conv->BN->neuron
nodes straight from torch modules (ONNX is not available to this build).

Pass order (optimize_ir, sengine/optimizer.py:24-59, restricted to this path):
  fold_batchnorm -> detect_fusion_groups -> mark_sparsity -> assign_kernels
"""
from __future__ import annotations

import numpy as np

from .ir import (BoundType, ConvParams, EngineIR, FusionGroup, KernelVariant, Node, NeuronParams, NeuronType,
                 OpType, TensorLayout, WeightInfo)
from .sparsity import fold_batchnorm as _fold_vectors
from .sparsity import validate_2_4_pattern

_TRANSPARENT = {OpType.Reshape, OpType.Transpose, OpType.Identity, OpType.Flatten}
_NEURONS = {OpType.LIF, OpType.IF}


def fold_batchnorm(ir: EngineIR) -> int:
    """Fold each Conv->BatchNorm pair into conv.bn_scale / conv.bn_bias (float64 fold, fp32
    storage) and remove the BN node — sengine/optimizer.py:126-191.  Weights are unchanged."""
    removed = 0
    for bn in [n for n in ir.nodes.values() if n.op_type == OpType.BatchNorm]:
        preds = ir.predecessors(bn.id)
        if not preds:
            continue
        conv = ir.nodes[preds[0]]
        if conv.op_type != OpType.Conv2d:
            continue
        a = bn.extra_attrs
        names = [a.get("bn_scale_name"), a.get("bn_bias_name"), a.get("bn_mean_name"), a.get("bn_var_name")]
        if not all(n in ir.weights for n in names):
            continue
        cb = ir.weights.get(conv.bias_info.name) if conv.bias_info else None
        scale, bias = _fold_vectors(*(ir.weights[n] for n in names), a.get("epsilon", 1e-5), cb)
        conv.bn_scale = scale.tolist()
        conv.bn_bias = bias.tolist()
        ir.remove_node(bn.id)
        removed += 1
    return removed


def _neuron_after(ir: EngineIR, nid: int):
    cur = nid
    for _ in range(8):
        succ = ir.successors(cur)
        if len(succ) != 1:
            return None
        n = ir.nodes[succ[0]]
        if n.op_type in _NEURONS:
            return n
        if n.op_type not in _TRANSPARENT:
            return None
        cur = n.id
    return None


def detect_fusion_groups(ir: EngineIR) -> int:
    """Conv -> (transparent ops) -> LIF/IF chains become FusionGroups (optimizer.py:452-492)."""
    ir.fusion_groups.clear()
    for nid in ir.topo_order:
        node = ir.nodes[nid]
        if node.op_type != OpType.Conv2d or node.fusion_group_id >= 0:
            continue
        neuron = _neuron_after(ir, nid)
        if neuron is None or neuron.fusion_group_id >= 0:
            continue
        gid = len(ir.fusion_groups)
        ir.fusion_groups.append(FusionGroup(gid, nid, neuron_node_id=neuron.id,
                                            bn_scale=node.bn_scale, bn_bias=node.bn_bias))
        node.fusion_group_id = gid
        neuron.fusion_group_id = gid
    return len(ir.fusion_groups)


def mark_sparsity(ir: EngineIR) -> int:
    """Conv nodes whose weights pass the engine's 2:4 check (stems with C_in < 4 excluded)
    get sparse_weight=True — sengine/optimizer.py:526-553."""
    n = 0
    for node in ir.nodes.values():
        if node.op_type != OpType.Conv2d or node.weight_info is None:
            continue
        w = ir.weights.get(node.weight_info.name)
        if w is None:
            continue
        if node.conv_params and node.conv_params.in_channels < 4:
            node.sparse_weight = False
            continue
        if validate_2_4_pattern(np.asarray(w)):
            node.sparse_weight = True
            node.weight_info.is_sparse = True
            n += 1
    return n


def fused_eligible(node: Node, T: int) -> bool:
    """Shapes the gfx950 fused kernel takes (C_in % 64, C_out % 64, groups 1, T in 1/2/4/8)."""
    cp = node.conv_params
    return (cp is not None and cp.groups == 1 and cp.in_channels % 64 == 0 and cp.out_channels % 64 == 0
            and T in (1, 2, 4, 8))


def dense_eligible(node: Node, T: int) -> bool:
    cp = node.conv_params
    return (cp is not None and cp.groups == 1 and cp.in_channels % 32 == 0 and cp.out_channels % 64 == 0
            and T in (1, 2, 4, 8))


def assign_kernels(ir: EngineIR) -> dict:
    """Kernel assignment (optimizer.py:839-864 + fusion_strategy.py:121-141 for this path):
      2:4 conv + neuron   -> conv: FusedSparseConvBNLIF (COMPUTE), neuron: ZeroCost (absorbed)
      dense conv + neuron -> conv: TileLangConvBN / TileLangConv1x1BN, neuron: CUDAVec4LIF / CUDAVec4IF
      other convs         -> CuDNNConv (not provided by this build)
    The anchor carries extra_attrs fusion_slice ('Conv2d+LIF' / 'Conv2d+IF') and absorbed_nids."""
    stats = {"fused": 0, "dense": 0, "unsupported": 0}
    T = ir.T
    for fg in ir.fusion_groups:
        conv, neuron = ir.nodes[fg.conv_node_id], ir.nodes[fg.neuron_node_id]
        if conv.sparse_weight and fused_eligible(conv, T):
            fg.variant = KernelVariant.FusedSparseConvBNLIF
            conv.assigned_kernel = KernelVariant.FusedSparseConvBNLIF
            conv.bound_type = BoundType.COMPUTE
            neuron.assigned_kernel = KernelVariant.ZeroCost
            neuron.bound_type = BoundType.ZERO
            conv.extra_attrs["fusion_slice"] = "Conv2d+" + ("LIF" if neuron.op_type == OpType.LIF else "IF")
            conv.extra_attrs["absorbed_nids"] = [neuron.id]
            stats["fused"] += 1
        elif dense_eligible(conv, T):
            cp = conv.conv_params
            one = cp.kernel_h == 1 and cp.kernel_w == 1
            conv.assigned_kernel = KernelVariant.TileLangConv1x1BN if one else KernelVariant.TileLangConvBN
            conv.bound_type = BoundType.COMPUTE
            neuron.assigned_kernel = (KernelVariant.CUDAVec4LIF if neuron.op_type == OpType.LIF
                                      else KernelVariant.CUDAVec4IF)
            neuron.bound_type = BoundType.MEMORY
            fg.variant = conv.assigned_kernel
            stats["dense"] += 1
        else:
            conv.assigned_kernel = KernelVariant.CuDNNConv
            neuron.assigned_kernel = KernelVariant.StandaloneLIF
            stats["unsupported"] += 1
        conv.layout = TensorLayout.NHWC
    return stats


def optimize_ir(ir: EngineIR) -> dict:
    """The hot-path subset of sengine's optimize_ir pipeline."""
    folded = fold_batchnorm(ir)
    groups = detect_fusion_groups(ir)
    sparse = mark_sparsity(ir)
    stats = assign_kernels(ir)
    stats.update(folded=folded, groups=groups, sparse=sparse)
    return stats


# --------------------------------------------------------------------------------------
# Front end: Conv2d -> BatchNorm2d -> multi-step neuron, straight from torch modules
# --------------------------------------------------------------------------------------

def add_conv_bn_neuron(ir: EngineIR, name: str, x_name: str, x_shape, conv, bn, neuron: str = "lif",
                       tau: float = 2.0, v_threshold: float = 1.0, v_reset=0.0) -> str:
    """Append Conv -> BN -> LIF/IF nodes for torch modules `conv` (nn.Conv2d) and `bn`
    (nn.BatchNorm2d) reading tensor `x_name` of NCHW shape x_shape = (T*B, C, H, W).
    v_reset=None means soft reset.  Returns the neuron's output tensor name."""
    N, C, H, W = x_shape
    kh, kw = conv.kernel_size
    sh, sw = conv.stride
    ph, pw = conv.padding
    dh, dw = conv.dilation
    OH = (H + 2 * ph - dh * (kh - 1) - 1) // sh + 1
    OW = (W + 2 * pw - dw * (kw - 1) - 1) // sw + 1
    out_shape = (N, conv.out_channels, OH, OW)
    wname = f"{name}.weight"
    ir.weights[wname] = conv.weight.detach().float().cpu().numpy()
    cnode = Node(0, f"{name}.conv", OpType.Conv2d, input_names=[x_name], output_names=[f"{name}.conv_out"],
                 input_shapes=[tuple(x_shape)], output_shapes=[out_shape],
                 conv_params=ConvParams(conv.in_channels, conv.out_channels, kh, kw, sh, sw, ph, pw, dh, dw, conv.groups),
                 weight_info=WeightInfo(wname, tuple(conv.weight.shape)))
    if conv.bias is not None:
        ir.weights[f"{name}.bias"] = conv.bias.detach().float().cpu().numpy()
        cnode.bias_info = WeightInfo(f"{name}.bias", tuple(conv.bias.shape))
    ir.add_node(cnode)
    names = {}
    for key, t in (("bn_scale_name", bn.weight), ("bn_bias_name", bn.bias), ("bn_mean_name", bn.running_mean),
                   ("bn_var_name", bn.running_var)):
        nm = f"{name}.bn.{key[3:-5]}"
        ir.weights[nm] = t.detach().float().cpu().numpy()
        names[key] = nm
    bnode = Node(0, f"{name}.bn", OpType.BatchNorm, input_names=[f"{name}.conv_out"],
                 output_names=[f"{name}.bn_out"], input_shapes=[out_shape], output_shapes=[out_shape],
                 extra_attrs=dict(names, epsilon=float(bn.eps)))
    ir.add_node(bnode)
    is_lif = neuron == "lif"
    npar = NeuronParams(NeuronType.LIF if is_lif else NeuronType.IF, ir.T, float(tau) if is_lif else 1.0,
                        float(v_threshold), 0.0 if v_reset is None else float(v_reset), v_reset is not None)
    nnode = Node(0, f"{name}.sn", OpType.LIF if is_lif else OpType.IF, is_stateful=True,
                 input_names=[f"{name}.bn_out"], output_names=[f"{name}.spikes"], input_shapes=[out_shape],
                 output_shapes=[out_shape], neuron_params=npar)
    ir.add_node(nnode)
    return f"{name}.spikes"
