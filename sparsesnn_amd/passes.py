"""Graph passes that select the fused 2:4 operator (the hot-path part of sengine/optimizer.py
and sengine/fusion_strategy.py), plus a small front end that builds Conv->BN->neuron
nodes straight from torch modules (ONNX is not available to this build).

Pass order (optimize_ir, sengine/optimizer.py:24-59, restricted to this path):
  fold_batchnorm -> detect_fusion_groups -> mark_sparsity -> assign_kernels
  -> fuse_stem -> absorb_residual_add -> absorb_membrane_shortcut -> assign_real_convs
  -> fuse_head -> assign_pools -> annotate_planes
(the passes after assign_kernels play the role of the reference's slicer for the
network-level nodes, sengine/fusion_strategy.py:28-193 / graph_slicer.py:43-182).
"""
from __future__ import annotations

import numpy as np

from .ir import (BoundType, ConvParams, EngineIR, FusionGroup, KernelVariant, Node, NeuronParams, NeuronType,
                 OpType, TensorLayout, WeightInfo)
from .sparsity import fold_batchnorm as _fold_vectors
from .sparsity import validate_2_4_pattern

_TRANSPARENT = {OpType.Reshape, OpType.Transpose, OpType.Identity, OpType.Flatten}
_NEURONS = {OpType.LIF, OpType.IF, OpType.MS}


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
            conv.extra_attrs["fusion_slice"] = "Conv2d+" + neuron.op_type.name
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


def _single_consumer(ir: EngineIR, nid: int):
    succ = ir.successors(nid)
    return ir.nodes[succ[0]] if len(succ) == 1 else None


def fuse_stem(ir: EngineIR) -> int:
    """Dense stem convs (C_in < 4: never 2:4 along C_in, optimizer.py:540-543) feeding
    Tile (repeat over T) -> LIF/IF/MS [-> MaxPool] run as one TileLangStemConvBN launch: the conv
    + BN once per image, the neuron over the T repeats and the spike max-pool from the same
    workgroup (the reference computes conv1/bn1 before repeating, models/sewresnet.py:199-201).
    The absorbed nodes become ZeroCost; extra_attrs: fusion_slice, absorbed_nids,
    fused_output (the tensor the launch writes).  When the repeated real-valued output has other
    readers besides the neuron (MS-ResNet's first shortcut, models/msresnet.py:111), the launch
    also stores it, once per image: extra_attrs real_output (that tensor)."""
    n = 0
    for nid in list(ir.topo_order):
        conv = ir.nodes[nid]
        if conv.op_type != OpType.Conv2d or conv.fusion_group_id >= 0 or conv.conv_params is None:
            continue
        if conv.conv_params.in_channels >= 4 or conv.conv_params.groups != 1 or conv.bn_scale is None:
            continue
        tile = _single_consumer(ir, nid)
        if tile is None or tile.op_type != OpType.Tile:
            continue
        readers = [ir.nodes[c] for c in ir.successors(tile.id)]
        neurons = [r for r in readers if r.op_type in _NEURONS]
        if len(neurons) != 1:
            continue
        neuron = neurons[0]
        real_out = tile.output_names[0] if len(readers) > 1 else None
        absorbed, pattern, out = [tile.id, neuron.id], ["Conv2d", "Tile", neuron.op_type.name], neuron.output_names[0]
        pool = _single_consumer(ir, neuron.id)
        if pool is not None and pool.op_type == OpType.MaxPool and real_out is None:
            absorbed.append(pool.id)
            pattern.append("MaxPool")
            out = pool.output_names[0]
        if real_out is not None:
            conv.extra_attrs["real_output"] = real_out
        conv.assigned_kernel = KernelVariant.TileLangStemConvBN
        conv.bound_type = BoundType.COMPUTE
        conv.layout = TensorLayout.NHWC
        conv.extra_attrs.update(fusion_slice="+".join(pattern), absorbed_nids=absorbed, fused_output=out,
                                neuron_nid=neuron.id)
        for a in absorbed:
            ir.nodes[a].assigned_kernel = KernelVariant.ZeroCost
            ir.nodes[a].bound_type = BoundType.ZERO
        n += 1
    return n


def _fused_anchor_of(ir: EngineIR, tensor: str):
    """The fused conv anchor whose absorbed neuron writes `tensor` (None otherwise)."""
    prod = ir._producer.get(tensor)
    if prod is None:
        return None
    node = ir.nodes[prod]
    if node.op_type not in _NEURONS or node.fusion_group_id < 0:
        return None
    anchor = ir.nodes[ir.fusion_groups[node.fusion_group_id].conv_node_id]
    if anchor.assigned_kernel != KernelVariant.FusedSparseConvBNLIF or "residual_input" in anchor.extra_attrs:
        return None
    return anchor


def absorb_residual_add(ir: EngineIR) -> int:
    """SEW 'ADD' (models/sewresnet.py:58-59) into the epilogue of the fused conv whose neuron
    feeds it -- the reference slicer's Conv2d+LIF+Add slice with one external residual input
    (graph_slicer.py:109-178, fusion_strategy.py:135-138).  Of two fused producers the one
    later in topological order absorbs the Add, so the residual exists when it runs.  The
    anchor records residual_nid (producer of the residual), residual_input (its tensor) and
    fused_output (the Add's output)."""
    order = {nid: i for i, nid in enumerate(ir.topo_order)}
    n = 0
    for nid in list(ir.topo_order):
        add = ir.nodes[nid]
        if add.op_type != OpType.Add or len(add.input_names) != 2 or add.assigned_kernel != KernelVariant.ZeroCost:
            continue
        cands = []
        for k, t in enumerate(add.input_names):
            anchor = _fused_anchor_of(ir, t)
            if anchor is not None and len(ir._consumers.get(t, [])) == 1:
                cands.append((order[anchor.id], k, anchor))
        if not cands:
            continue
        _, k, anchor = max(cands, key=lambda c: c[0])
        res_t = add.input_names[1 - k]
        anchor.extra_attrs["absorbed_nids"] = list(anchor.extra_attrs.get("absorbed_nids", [])) + [add.id]
        anchor.extra_attrs["fusion_slice"] = anchor.extra_attrs.get("fusion_slice", "Conv2d+LIF") + "+Add"
        anchor.extra_attrs["residual_nid"] = ir._producer.get(res_t)
        anchor.extra_attrs["residual_input"] = res_t
        anchor.extra_attrs["fused_output"] = add.output_names[0]
        add.assigned_kernel = KernelVariant.ZeroCost
        add.bound_type = BoundType.ZERO
        add.extra_attrs["absorbed_into"] = anchor.id
        n += 1
    return n


def fuse_head(ir: EngineIR) -> int:
    """GlobalAvgPool -> Flatten -> TemporalMean -> Gemm (avgpool, flatten, x.mean(0), fc;
    models/sewresnet.py:206-210) or TemporalMean -> GlobalAvgPool -> Flatten -> Gemm
    (models/msresnet.py:153-161) as one CuBLASGemm launch on the spike counts: the pooled
    means are integer counts times 1/(HW*T) in either order, so the pool and mean run exactly
    on integers before the Linear.  The Gemm node anchors it (fusion_slice, absorbed_nids --
    the chain from the Gemm back, its first op last -- and head_input)."""
    n = 0
    for nid in list(ir.topo_order):
        gemm = ir.nodes[nid]
        if gemm.op_type != OpType.Gemm:
            continue
        chain, cur = [], gemm
        while True:
            preds = ir.predecessors(cur.id)
            if len(preds) != 1:
                break
            p = ir.nodes[preds[0]]
            if p.op_type in (OpType.TemporalMean, OpType.Flatten, OpType.Reshape, OpType.GlobalAvgPool):
                chain.append(p)
                cur = p
            else:
                break
        kinds = {c.op_type for c in chain}
        if OpType.GlobalAvgPool not in kinds or OpType.TemporalMean not in kinds:
            continue
        first = chain[-1]
        gemm.assigned_kernel = KernelVariant.CuBLASGemm
        gemm.bound_type = BoundType.MEMORY
        gemm.extra_attrs.update(fusion_slice="+".join([c.op_type.name for c in reversed(chain)] + ["Gemm"]),
                                absorbed_nids=[c.id for c in chain], head_input=first.input_names[0])
        for c in chain:
            c.assigned_kernel = KernelVariant.ZeroCost
            c.bound_type = BoundType.ZERO
        n += 1
    return n


def absorb_membrane_shortcut(ir: EngineIR) -> int:
    """MS-ResNet's block output out = conv_bn2 + shortcut (models/msresnet.py:107-112) with the
    next neuron on it (the next block's sn1, or sn_out) into one launch: the 2:4 conv + folded
    BN whose output feeds only the Add becomes a FusedSparseConvBNLIF anchor that adds the
    real-valued shortcut, stores the sum (the next block's real-valued input) and fires the
    neuron -- the reference engine's Add+LIF fusion (TileLangFusedAddLIF,
    sengine/kernels/add_lif_fused.py:20-75) with the conv in front of it.  extra_attrs:
    shortcut_input (the Add's other input), real_output (the Add's output), fused_output (the
    neuron's spikes), absorbed_nids [Add, neuron]."""
    n = 0
    for nid in list(ir.topo_order):
        add = ir.nodes[nid]
        if add.op_type != OpType.Add or len(add.input_names) != 2 or add.assigned_kernel != KernelVariant.ZeroCost:
            continue
        if any(add.id in a.extra_attrs.get("absorbed_nids", []) for a in ir.nodes.values()):
            continue
        y = add.output_names[0]
        neurons = [ir.nodes[c] for c in ir._consumers.get(y, []) if ir.nodes[c].op_type in _NEURONS]
        if len(neurons) != 1:
            continue
        neuron = neurons[0]
        for k in (0, 1):
            pid = ir._producer.get(add.input_names[k])
            conv = ir.nodes.get(pid) if pid is not None else None
            if (conv is None or conv.op_type != OpType.Conv2d or conv.fusion_group_id >= 0 or conv.bn_scale is None
                    or not conv.sparse_weight or conv.assigned_kernel != KernelVariant.ZeroCost
                    or not fused_eligible(conv, ir.T) or len(ir._consumers.get(add.input_names[k], [])) != 1):
                continue
            conv.assigned_kernel = KernelVariant.FusedSparseConvBNLIF
            conv.bound_type = BoundType.COMPUTE
            conv.layout = TensorLayout.NHWC
            conv.extra_attrs.update(fusion_slice="Conv2d+Add+" + neuron.op_type.name, absorbed_nids=[add.id, neuron.id],
                                    shortcut_input=add.input_names[1 - k], real_output=y,
                                    fused_output=neuron.output_names[0], neuron_nid=neuron.id)
            for a in (add, neuron):
                a.assigned_kernel = KernelVariant.ZeroCost
                a.bound_type = BoundType.ZERO
            n += 1
            break
    return n


def _real_tensors(ir: EngineIR) -> set:
    """Real-valued (fp32) tensors the launches write: stems' kept outputs and membrane-shortcut sums."""
    return {n.extra_attrs["real_output"] for n in ir.nodes.values() if "real_output" in n.extra_attrs}


def assign_real_convs(ir: EngineIR) -> int:
    """1x1 convs + folded BN on a real-valued tensor (MS-ResNet's TDBN shortcut of the block
    input, models/msresnet.py:100-105) run as fp32 1x1 Conv+BN launches: TileLangConv1x1BN with
    extra_attrs real_input (the products of real activations are not exact in fp16, so the
    spike kernels do not apply)."""
    real = _real_tensors(ir)
    n = 0
    for node in ir.nodes.values():
        cp = node.conv_params
        if node.op_type != OpType.Conv2d or node.assigned_kernel != KernelVariant.ZeroCost or cp is None:
            continue
        if node.bn_scale is None or node.input_names[0] not in real or cp.kernel_h != 1 or cp.kernel_w != 1 or \
                cp.pad_h != 0 or cp.pad_w != 0 or cp.groups != 1:
            continue
        node.assigned_kernel = KernelVariant.TileLangConv1x1BN
        node.bound_type = BoundType.MEMORY
        node.layout = TensorLayout.NHWC
        node.extra_attrs["real_input"] = True
        n += 1
    return n


def assign_pools(ir: EngineIR) -> int:
    """Max-pools not absorbed by a stem run as CuDNNPool on spike bits (OR of the window)."""
    n = 0
    for node in ir.nodes.values():
        if node.op_type == OpType.MaxPool and node.assigned_kernel == KernelVariant.ZeroCost and \
                not any(node.id in a.extra_attrs.get("absorbed_nids", []) for a in ir.nodes.values()):
            node.assigned_kernel = KernelVariant.CuDNNPool
            node.bound_type = BoundType.MEMORY
            node.layout = TensorLayout.NHWC
            n += 1
    return n


def annotate_planes(ir: EngineIR) -> int:
    """Integer range of every activation: spikes are 0/1, a fused SEW add yields
    max(residual) + 1, max-pool keeps its input's range.  Fused convs record in_planes (the
    bit planes of their input, which multiply the reduction, sparsity.expand_planes) and
    out_planes; residual sums above 31 (5 planes) are rejected."""
    vmax: dict = {}
    for nid in ir.topo_order:
        node = ir.nodes[nid]
        kv = node.assigned_kernel
        if node.op_type in _NEURONS:
            for o in node.output_names:
                vmax[o] = 1
        if kv == KernelVariant.FusedSparseConvBNLIF:
            inp = node.input_names[0]
            node.extra_attrs["in_planes"] = max(1, int(vmax.get(inp, 1)).bit_length())
            if "residual_input" in node.extra_attrs:
                m = int(vmax.get(node.extra_attrs["residual_input"], 1)) + 1
                if m > 31:
                    raise ValueError(f"{node.name}: residual sums up to {m} need more than 5 bit planes")
                vmax[node.extra_attrs["fused_output"]] = m
                node.extra_attrs["res_planes"] = max(1, int(m - 1).bit_length())
                node.extra_attrs["out_planes"] = m.bit_length()
            else:
                node.extra_attrs["out_planes"] = 1
        elif node.op_type in (OpType.MaxPool, OpType.Flatten, OpType.Reshape, OpType.Identity):
            for o in node.output_names:
                vmax[o] = vmax.get(node.input_names[0], 1)
        elif kv == KernelVariant.TileLangStemConvBN:
            vmax[node.extra_attrs["fused_output"]] = 1
        elif kv == KernelVariant.CuBLASGemm and "head_input" in node.extra_attrs:
            node.extra_attrs["in_planes"] = max(1, int(vmax.get(node.extra_attrs["head_input"], 1)).bit_length())
    return len(vmax)


def optimize_ir(ir: EngineIR) -> dict:
    """The hot-path subset of sengine's optimize_ir pipeline, plus the network-level fusions
    the generic runtime serves (stem, SEW add, head, pools)."""
    folded = fold_batchnorm(ir)
    groups = detect_fusion_groups(ir)
    sparse = mark_sparsity(ir)
    stats = assign_kernels(ir)
    stems = fuse_stem(ir)
    adds = absorb_residual_add(ir)
    shortcuts = absorb_membrane_shortcut(ir)
    real_convs = assign_real_convs(ir)
    heads = fuse_head(ir)
    pools = assign_pools(ir)
    annotate_planes(ir)
    stats.update(folded=folded, groups=groups, sparse=sparse, stems=stems, adds=adds, heads=heads, pools=pools,
                 shortcuts=shortcuts, real_convs=real_convs)
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
