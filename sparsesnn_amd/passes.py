"""Graph passes that select the fused 2:4 operator (the hot-path part of sengine/optimizer.py
and sengine/fusion_strategy.py), plus a small front end that builds Conv->BN->neuron
nodes straight from torch modules (ONNX is not available to this build).

Pass order (optimize_ir, sengine/optimizer.py:24-59, restricted to this path):
  lower_linears -> fold_batchnorm -> detect_fusion_groups -> mark_sparsity -> pad_channels
  -> assign_kernels -> fuse_stem -> absorb_residual_add -> absorb_membrane_shortcut
  -> assign_real_convs -> merge_sibling_convs -> assign_attention -> fuse_head -> assign_pools
  -> annotate_planes
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


def lower_linears(ir: EngineIR) -> int:
    """Token Linears (OpType.Linear, weight (out, in) as nn.Linear holds it, optional bias) over a
    (T*B, C, N, 1) token grid become 1x1 Conv2d nodes over that grid: y[t, :, n] = W x[t, :, n] + b
    is the 1x1 convolution with weight W[:, :, None, None] and that bias (the reference fuses
    Linear + BatchNorm1d + LIF the same way, TileLangLinearBNLIF, sengine/ir.py:72-74).  The
    BatchNorm1d that follows is the per-channel affine fold_batchnorm folds; the Linear bias
    goes into it as the conv bias.  Returns the number of nodes lowered."""
    n = 0
    for node in ir.nodes.values():
        if node.op_type != OpType.Linear or node.weight_info is None:
            continue
        w = np.asarray(ir.weights[node.weight_info.name])
        shp = tuple(node.input_shapes[0]) if node.input_shapes else ()
        if w.ndim != 2 or len(shp) != 4 or shp[3] != 1 or shp[1] != w.shape[1]:
            raise ValueError(f"node {node.name}: a Linear over a (T*B, C, N, 1) token grid with a 2-D weight "
                             f"is served, got input {shp} and weight {w.shape}")
        w4 = w[:, :, None, None]
        ir.weights[node.weight_info.name] = w4
        node.weight_info.shape = tuple(w4.shape)
        node.op_type = OpType.Conv2d
        node.conv_params = ConvParams(int(w.shape[1]), int(w.shape[0]), 1, 1, 1, 1, 0, 0)
        node.extra_attrs["lowered_from"] = "Linear"
        n += 1
    return n


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


def _pad_to(c: int, multiple: int) -> int:
    return -(-c // multiple) * multiple


def _pad_weight(ir: EngineIR, node: Node, axis: int, size: int):
    """Zero-pad the node's weight along `axis` (0 = C_out, 1 = C_in) to `size`, stored under a
    name of its own (the original array is left alone)."""
    w = np.asarray(ir.weights[node.weight_info.name])
    pad = [(0, 0)] * w.ndim
    pad[axis] = (0, size - w.shape[axis])
    name = node.weight_info.name if node.weight_info.name.endswith("#padded") else node.weight_info.name + "#padded"
    ir.weights[name] = np.pad(w, pad)
    node.weight_info = WeightInfo(name, tuple(ir.weights[name].shape), node.weight_info.is_sparse)


def _with_channels(shape, c):
    return (shape[0], c) + tuple(shape[2:])


def pad_channels(ir: EngineIR, multiple: int = 64) -> int:
    """Pad the output channels of a Conv -> BN [-> Tile] -> neuron chain to a multiple of 64
    (the fused kernels' channel blocking; Spikformer's SPS has embed/8 = 48 and embed/4 = 96
    channels, models/spikformer.py:159-165) with zero weights and a zero BN affine: the padded
    channels' input is 0 every step, so a neuron with V_th > max(0, V_reset) never fires there.
    Their spikes flow through max-pools into convs only, whose input channels get matching zero
    weight columns (a group of four zeros keeps the
    kernels' rule of at most two nonzeros per group).  Chains whose spikes reach anything else
    are left alone.  Shapes along the way are updated, and each reader records its real input
    channel count (extra_attrs["in_channels_real"]).  Returns the number of convs padded."""
    n = 0
    for nid in list(ir.topo_order):
        conv = ir.nodes[nid]
        cp = conv.conv_params
        if conv.op_type != OpType.Conv2d or cp is None or cp.groups != 1 or conv.bn_scale is None or \
                conv.weight_info is None or cp.out_channels % multiple == 0:
            continue
        path = []
        nxt = _single_consumer(ir, nid)
        if nxt is not None and nxt.op_type == OpType.Tile:
            path.append(nxt)
            nxt = _single_consumer(ir, nxt.id)
        if nxt is None or nxt.op_type not in _NEURONS or nxt.neuron_params is None:
            continue
        npar = nxt.neuron_params
        if not npar.v_threshold > max(0.0, npar.v_reset if npar.hard_reset else 0.0):
            continue
        path.append(nxt)
        carriers, readers, frontier, ok = [], [], [nxt.id], True
        while frontier and ok:
            cur = frontier.pop()
            for sid in ir.successors(cur):
                sn = ir.nodes[sid]
                if sn.op_type in (OpType.MaxPool, OpType.Identity):
                    carriers.append(sn)
                    frontier.append(sid)
                elif sn.op_type == OpType.Conv2d and sn.conv_params is not None and sn.conv_params.groups == 1 \
                        and sn.weight_info is not None and len(sn.input_names) == 1:
                    readers.append(sn)
                else:
                    ok = False
                    break
        if not ok or not readers:
            continue
        real = cp.out_channels
        P = _pad_to(real, multiple)
        _pad_weight(ir, conv, 0, P)
        extra = [0.0] * (P - cp.out_channels)
        conv.bn_scale = list(conv.bn_scale) + extra
        conv.bn_bias = list(conv.bn_bias) + extra
        cp.out_channels = P
        conv.output_shapes = [_with_channels(conv.output_shapes[0], P)]
        for m in path + carriers:
            m.input_shapes = [_with_channels(s, P) for s in m.input_shapes]
            m.output_shapes = [_with_channels(s, P) for s in m.output_shapes]
        for r in readers:
            _pad_weight(ir, r, 1, P)
            r.conv_params.in_channels = P
            r.input_shapes = [_with_channels(r.input_shapes[0], P)] + list(r.input_shapes[1:])
            r.extra_attrs["in_channels_real"] = real  # the rest are zero padding (paired-tail form)
        conv.extra_attrs["padded_from"] = int(P - len(extra))
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


def merge_sibling_convs(ir: EngineIR, round_to: int = 256) -> int:
    """Fused 1x1 convs that read the same tensor with the same shape and neuron and no residual
    (Spikformer's q, k and v Linears, models/spikformer.py:103-125) run as one launch over their
    weights concatenated along C_out -- the input is read once instead of once per conv -- with
    the spike bits split back into one plane per conv (sengine_amd_fused_sparse_conv_bn_lif_split).
    The concatenation is zero-padded to a multiple of `round_to` output channels (zero weights
    and a zero BN affine: never fire; 256 = the persistent 1x1 kernel's four-wave super-block).
    The first conv anchors the launch: extra_attrs merged_nids (the convs, in order),
    merged_weight (the concatenated weight's name in ir.weights), merged_bn (scale, bias lists),
    merged_outputs (each conv's spike tensor) and split_channels; the other convs and their
    neurons are absorbed (ZeroCost).  Returns the number of merged launches."""
    groups: dict = {}
    for nid in ir.topo_order:
        n = ir.nodes[nid]
        ea = n.extra_attrs
        cp = n.conv_params
        if n.assigned_kernel != KernelVariant.FusedSparseConvBNLIF or cp is None or \
                any(k in ea for k in ("residual_input", "shortcut_input", "merged_nids")):
            continue
        if (cp.kernel_h, cp.kernel_w, cp.stride_h, cp.stride_w, cp.pad_h, cp.pad_w) != (1, 1, 1, 1, 0, 0) or \
                cp.out_channels % 64:
            continue
        absorbed = ea.get("absorbed_nids", [])
        if len(absorbed) != 1:
            continue
        neuron = ir.nodes[absorbed[0]]
        np_ = neuron.neuron_params
        key = (n.input_names[0], cp.in_channels, cp.out_channels, tuple(n.input_shapes[0]), neuron.op_type,
               None if np_ is None else (np_.tau, np_.v_threshold, np_.v_reset, np_.hard_reset))
        groups.setdefault(key, []).append((n, neuron))
    merged = 0
    for key, members in groups.items():
        if len(members) < 2:
            continue
        anchor = members[0][0]
        cout = anchor.conv_params.out_channels
        total = _pad_to(len(members) * cout, round_to)
        ws = [np.asarray(ir.weights[c.weight_info.name], dtype=np.float32) for c, _ in members]
        w = np.zeros((total,) + ws[0].shape[1:], np.float32)
        w[:len(members) * cout] = np.concatenate(ws)
        zeros = [0.0] * (total - len(members) * cout)
        wname = anchor.name + ".merged.weight"
        ir.weights[wname] = w
        absorbed = [members[0][1].id]
        for c, nr in members[1:]:
            absorbed += [c.id, nr.id]
            for x in (c, nr):
                x.assigned_kernel = KernelVariant.ZeroCost
                x.bound_type = BoundType.ZERO
        anchor.extra_attrs.update(
            merged_nids=[c.id for c, _ in members], merged_weight=wname, split_channels=cout,
            merged_bn=(sum((list(c.bn_scale) for c, _ in members), []) + zeros,
                       sum((list(c.bn_bias) for c, _ in members), []) + zeros),
            merged_outputs=[nr.output_names[0] for _, nr in members], merged_out_channels=total,
            absorbed_nids=absorbed,
            fusion_slice="Split(" + ",".join("Conv2d+" + nr.op_type.name for _, nr in members) + ")")
        merged += 1
    return merged


def assign_attention(ir: EngineIR) -> int:
    """FusedAttention nodes of the Spikformer variant run as FusedSpikformerAttn (the SSA core on
    spike bits: K^T V per head, then Q (K^T V) * scale and the attention LIF in one more launch);
    other variants are not served here and raise."""
    n = 0
    for node in ir.nodes.values():
        if node.op_type != OpType.FusedAttention:
            continue
        ap = node.attention_params
        if ap is None or ap.variant != "spikformer" or len(node.input_names) != 3:
            raise ValueError(f"node {node.name}: only the Spikformer attention core (q, k, v) is served")
        node.assigned_kernel = KernelVariant.FusedSpikformerAttn
        node.bound_type = BoundType.COMPUTE
        node.layout = TensorLayout.NHWC
        n += 1
    return n


def annotate_planes(ir: EngineIR, int_stream: str = "planes") -> int:
    """Integer range of every activation: spikes are 0/1, a fused SEW add yields
    max(residual) + 1, max-pool keeps its input's range.  Fused convs record in_planes (the
    bit planes of their input, which multiply the reduction, sparsity.expand_planes) and
    out_planes; residual sums above 31 (5 planes) are rejected.

    int_stream 'f16': integer activations (ranges above 1) are stored as fp16 integers instead
    -- the reference's own representation of the residual stream -- exact up to 2048.  Their
    readers record in_planes 0 (an fp16 input, K = C_in) and res_planes 0; their writers
    out_planes 0 (fp16 output)."""
    if int_stream not in ("planes", "f16"):
        raise ValueError("int_stream must be 'planes' or 'f16'")
    f16 = int_stream == "f16"
    ir.int_stream = int_stream
    vmax: dict = {}

    def planes_of(t):
        m = int(vmax.get(t, 1))
        return 0 if (f16 and m > 1) else max(1, m.bit_length())

    for nid in ir.topo_order:
        node = ir.nodes[nid]
        kv = node.assigned_kernel
        if node.op_type in _NEURONS or node.op_type == OpType.FusedAttention:
            for o in node.output_names:
                vmax[o] = 1
        if kv == KernelVariant.FusedSparseConvBNLIF:
            inp = node.input_names[0]
            node.extra_attrs["in_planes"] = planes_of(inp)
            if "residual_input" in node.extra_attrs:
                res = node.extra_attrs["residual_input"]
                m = int(vmax.get(res, 1)) + 1
                if f16 and m >= 2048:
                    raise ValueError(f"{node.name}: residual sums up to {m} exceed fp16's exact integers")
                if not f16 and m > 31:
                    raise ValueError(f"{node.name}: residual sums up to {m} need more than 5 bit planes")
                vmax[node.extra_attrs["fused_output"]] = m
                node.extra_attrs["res_planes"] = planes_of(res)
                node.extra_attrs["out_planes"] = 0 if f16 else m.bit_length()
            else:
                node.extra_attrs["out_planes"] = 1
        elif node.op_type in (OpType.MaxPool, OpType.Flatten, OpType.Reshape, OpType.Identity):
            for o in node.output_names:
                vmax[o] = vmax.get(node.input_names[0], 1)
        elif kv == KernelVariant.TileLangStemConvBN:
            vmax[node.extra_attrs["fused_output"]] = 1
        elif kv == KernelVariant.CuBLASGemm and "head_input" in node.extra_attrs:
            node.extra_attrs["in_planes"] = planes_of(node.extra_attrs["head_input"])
    return len(vmax)


def optimize_ir(ir: EngineIR, int_stream: str = "planes") -> dict:
    """The hot-path subset of sengine's optimize_ir pipeline, plus the network-level fusions
    the generic runtime serves (stem, SEW add, membrane shortcut, merged siblings, attention,
    head, pools).  int_stream: how integer activations (residual sums) are stored, annotate_planes."""
    linears = lower_linears(ir)
    folded = fold_batchnorm(ir)
    groups = detect_fusion_groups(ir)
    sparse = mark_sparsity(ir)
    padded = pad_channels(ir)
    stats = assign_kernels(ir)
    stems = fuse_stem(ir)
    adds = absorb_residual_add(ir)
    shortcuts = absorb_membrane_shortcut(ir)
    real_convs = assign_real_convs(ir)
    merged = merge_sibling_convs(ir)
    attention = assign_attention(ir)
    heads = fuse_head(ir)
    pools = assign_pools(ir)
    annotate_planes(ir, int_stream)
    stats.update(folded=folded, groups=groups, sparse=sparse, stems=stems, adds=adds, heads=heads, pools=pools,
                 shortcuts=shortcuts, real_convs=real_convs, linears=linears, padded=padded, merged=merged,
                 attention=attention)
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
