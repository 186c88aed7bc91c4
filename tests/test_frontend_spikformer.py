"""CPU: the Spikformer front end (frontend.spikformer_ir) and the passes that map it onto the
generic engine's launches -- lower_linears, pad_channels, merge_sibling_convs, assign_attention
and annotate_planes' fp16 stream -- against the structure of models/spikformer.py:59-288 and
the launch sequence of the hand-wired SpikformerEngine."""
import numpy as np
import pytest

from sparsesnn_amd import frontend, passes
from sparsesnn_amd.compiler import SparseKernelCompiler, SpikeHeadKernel, SpikingSelfAttentionKernel
from sparsesnn_amd.ir import (ConvParams, EngineIR, KernelVariant, Node, NeuronParams, NeuronType, OpType,
                              WeightInfo)
from sparsesnn_amd.runtime import CUDAGraphEngine
from sparsesnn_amd.spikformer import random_params

EMBED, HEADS, DEPTH = 128, 2, 3


def _ir(int_stream="f16", embed=EMBED, depth=DEPTH, hw=(32, 32)):
    p = random_params(3, embed=embed, depth=depth, num_classes=10)
    ir = frontend.spikformer_ir(p, T=4, batch=2, in_hw=hw, heads=HEADS)
    stats = passes.optimize_ir(ir, int_stream=int_stream)
    return p, ir, stats


def _launches(ir):
    eng = CUDAGraphEngine()
    launches, aliases, shapes = eng._analyse(ir, ir.topo_order)
    return eng, eng._order(launches, aliases, ir.topo_order), aliases, shapes


def _node(ir, name):
    return next(n for n in ir.nodes.values() if n.name == name)


def test_front_end_inventory():
    p = random_params(3, embed=EMBED, depth=DEPTH, num_classes=10)
    ir = frontend.spikformer_ir(p, T=4, batch=2, in_hw=(32, 32), heads=HEADS)
    ops_ = [n.op_type for n in ir.nodes.values()]
    assert ops_.count(OpType.Conv2d) == 5 and ops_.count(OpType.Linear) == 6 * DEPTH
    assert ops_.count(OpType.BatchNorm) == 5 + 6 * DEPTH
    assert ops_.count(OpType.LIF) == 5 + 6 * DEPTH  # attn_lif lives inside the attention node
    assert ops_.count(OpType.FusedAttention) == DEPTH and ops_.count(OpType.Add) == 1 + 2 * DEPTH
    assert ops_.count(OpType.MaxPool) == 2 and ops_.count(OpType.Tile) == 1
    core = _node(ir, "block.0.attn.core")
    ap = core.attention_params
    assert (ap.variant, ap.num_heads, ap.head_dim, ap.scale, ap.attn_lif_v_threshold) == \
        ("spikformer", HEADS, EMBED // HEADS, 0.125, 0.5)
    tok = _node(ir, "patch_embed.tokens")
    assert tok.output_shapes[0] == (8, EMBED, 64, 1)  # 32x32 -> two 3x3/2 pools -> 8x8 = 64 tokens


def test_passes_stats():
    _, ir, st = _ir()
    assert st["linears"] == 6 * DEPTH and st["folded"] == 5 + 6 * DEPTH
    assert st["padded"] == 2  # embed/8 and embed/4 channels (16, 32) -> 64
    assert st["fused"] == 4 + 6 * DEPTH and st["stems"] == 1 and st["pools"] == 2
    assert st["adds"] == 1 + 2 * DEPTH and st["merged"] == DEPTH and st["attention"] == DEPTH
    assert st["heads"] == 1 and st["shortcuts"] == 0 and st["real_convs"] == 0


def test_linears_lowered_to_token_grid_convs():
    p, ir, _ = _ir()
    fc1 = _node(ir, "block.1.mlp.fc1_linear")
    assert fc1.op_type == OpType.Conv2d and fc1.extra_attrs["lowered_from"] == "Linear"
    cp = fc1.conv_params
    assert (cp.in_channels, cp.out_channels, cp.kernel_h, cp.kernel_w) == (EMBED, 4 * EMBED, 1, 1)
    w = ir.weights[fc1.weight_info.name]
    assert w.shape == (4 * EMBED, EMBED, 1, 1)
    assert np.array_equal(w[:, :, 0, 0], p["block.1.mlp.fc1_linear.weight"].numpy())
    assert fc1.input_shapes[0] == (8, EMBED, 64, 1)


def test_sps_channels_padded():
    p, ir, _ = _ir()
    stem, c1, c2 = (_node(ir, n) for n in ("patch_embed.proj_conv", "patch_embed.proj_conv1",
                                            "patch_embed.proj_conv2"))
    assert stem.conv_params.out_channels == 64 and stem.extra_attrs["padded_from"] == EMBED // 8
    assert c1.conv_params.in_channels == 64 and c1.conv_params.out_channels == 64
    assert c2.conv_params.in_channels == 64 and c2.conv_params.out_channels == EMBED // 2
    w1 = ir.weights[c1.weight_info.name]
    src = p["patch_embed.proj_conv1.weight"].numpy()
    assert w1.shape == (64, 64, 3, 3)
    assert np.array_equal(w1[:EMBED // 4, :EMBED // 8], src)
    assert not w1[EMBED // 4:].any() and not w1[:, EMBED // 8:].any()
    assert c1.bn_scale[EMBED // 4:] == [0.0] * (64 - EMBED // 4) and c1.bn_bias[EMBED // 4:] == [0.0] * 32
    assert _node(ir, "patch_embed.proj_lif").output_shapes[0][1] == 64
    assert _node(ir, "patch_embed.repeat").output_shapes[0][1] == 64
    # the original arrays are untouched
    assert ir.weights["patch_embed.proj_conv1.weight"].shape == src.shape


def test_pad_channels_leaves_other_readers_alone():
    """A 48-channel neuron whose spikes reach an Add (not a conv) is not padded, nor one whose
    threshold is not above 0."""
    for vth, reader in ((1.0, OpType.Add), (0.0, OpType.Conv2d)):
        ir = EngineIR()
        rng = np.random.default_rng(0)
        ir.weights["c.w"] = rng.standard_normal((48, 64, 3, 3)).astype(np.float32)
        ir.weights["d.w"] = rng.standard_normal((64, 48, 1, 1)).astype(np.float32)
        ir.add_node(Node(0, "c", OpType.Conv2d, input_names=["x"], output_names=["c.out"],
                         input_shapes=[(8, 64, 4, 4)], output_shapes=[(8, 48, 4, 4)],
                         conv_params=ConvParams(64, 48, 3, 3, 1, 1, 1, 1), weight_info=WeightInfo("c.w", (48, 64, 3, 3)),
                         bn_scale=[1.0] * 48, bn_bias=[0.0] * 48))
        ir.add_node(Node(0, "n", OpType.LIF, input_names=["c.out"], output_names=["n.out"],
                         input_shapes=[(8, 48, 4, 4)], output_shapes=[(8, 48, 4, 4)],
                         neuron_params=NeuronParams(NeuronType.LIF, 4, 2.0, vth, 0.0, True)))
        if reader == OpType.Add:
            ir.add_node(Node(0, "a", OpType.Add, input_names=["n.out", "y"], output_names=["a.out"],
                             input_shapes=[(8, 48, 4, 4)], output_shapes=[(8, 48, 4, 4)]))
        else:
            ir.add_node(Node(0, "d", OpType.Conv2d, input_names=["n.out"], output_names=["d.out"],
                             input_shapes=[(8, 48, 4, 4)], output_shapes=[(8, 64, 4, 4)],
                             conv_params=ConvParams(48, 64, 1, 1), weight_info=WeightInfo("d.w", (64, 48, 1, 1))))
        assert passes.pad_channels(ir) == 0
        assert ir.nodes[0].conv_params.out_channels == 48 and ir.nodes[0].weight_info.name == "c.w"


def test_qkv_merged_into_one_split_launch():
    p, ir, _ = _ir()
    q = _node(ir, "block.2.attn.q_linear")
    ea = q.extra_attrs
    names = [ir.nodes[n].name for n in ea["merged_nids"]]
    assert names == [f"block.2.attn.{n}_linear" for n in "qkv"]
    assert ea["split_channels"] == EMBED and ea["merged_out_channels"] == 512  # 3 * 128 -> 256-multiple
    assert ea["fusion_slice"] == "Split(Conv2d+LIF,Conv2d+LIF,Conv2d+LIF)"
    w = ir.weights[ea["merged_weight"]]
    assert w.shape == (512, EMBED, 1, 1)
    for j, n in enumerate("qkv"):
        assert np.array_equal(w[j * EMBED:(j + 1) * EMBED, :, 0, 0], p[f"block.2.attn.{n}_linear.weight"].numpy())
    assert not w[3 * EMBED:].any()
    sc, bi = ea["merged_bn"]
    k = _node(ir, "block.2.attn.k_linear")
    assert len(sc) == 512 and sc[EMBED:2 * EMBED] == list(k.bn_scale) and sc[3 * EMBED:] == [0.0] * EMBED
    assert bi[2 * EMBED:3 * EMBED] == list(_node(ir, "block.2.attn.v_linear").bn_bias)
    assert k.assigned_kernel == KernelVariant.ZeroCost
    assert ea["merged_outputs"] == [f"block.2.attn.{n}_lif.out" for n in "qkv"]


def test_stream_annotation_f16_and_planes():
    _, ir, _ = _ir("f16")
    rpe, q, proj, fc1, fc2, head = (_node(ir, n) for n in (
        "patch_embed.rpe_conv", "block.0.attn.q_linear", "block.0.attn.proj_linear", "block.0.mlp.fc1_linear",
        "block.0.mlp.fc2_linear", "head"))
    assert (rpe.extra_attrs["in_planes"], rpe.extra_attrs["res_planes"], rpe.extra_attrs["out_planes"]) == (1, 1, 0)
    assert q.extra_attrs["in_planes"] == 0 and fc1.extra_attrs["in_planes"] == 0
    assert (proj.extra_attrs["res_planes"], proj.extra_attrs["out_planes"]) == (0, 0)
    assert (fc2.extra_attrs["in_planes"], fc2.extra_attrs["res_planes"]) == (1, 0)
    assert head.extra_attrs["in_planes"] == 0
    _, ir, _ = _ir("planes")
    rpe, q, proj, fc2, head = (_node(ir, n) for n in (
        "patch_embed.rpe_conv", "block.0.attn.q_linear", "block.0.attn.proj_linear", "block.0.mlp.fc2_linear",
        "head"))
    # the stream's range grows by 2 per block from 2 (rpe spike + pooled spike): planes as SpikformerEngine
    assert rpe.extra_attrs["out_planes"] == 2 and q.extra_attrs["in_planes"] == 2
    assert (proj.extra_attrs["res_planes"], proj.extra_attrs["out_planes"]) == (2, 2)
    assert fc2.extra_attrs["out_planes"] == 3
    assert head.extra_attrs["in_planes"] == (2 + 2 * DEPTH).bit_length()


def test_launch_sequence_matches_the_hand_wired_engine():
    """stem, conv1, conv2, pool, conv3, pool, rpe (+ add); per block q/k/v split, attention,
    proj (+ add), fc1, fc2 (+ add); head -- SpikformerEngine's order."""
    _, ir, _ = _ir()
    eng, launches, aliases, shapes = _launches(ir)
    kinds = [l.kind for l in launches]
    assert kinds == ["stem", "fused", "fused", "pool", "fused", "pool", "fused"] + \
        ["split", "attn", "fused", "fused", "fused"] * DEPTH + ["head"]
    split = launches[7]
    assert shapes[split.output] == (8, 4 * EMBED, 64, 1)  # four planes of 128 channels (the fourth: padding)
    attn = launches[8]
    assert [eng.sub[t] for t in attn.inputs] == [(0, 4), (1, 4), (2, 4)]
    assert all(aliases[t] == split.output for t in attn.inputs)


def test_kernel_objects():
    _, ir, _ = _ir()
    kernels = SparseKernelCompiler(ir, batch_size=2).compile_all()
    q = _node(ir, "block.0.attn.q_linear")
    spec = kernels[q.id].spec
    assert (spec.C_in, spec.C_out, spec.H, spec.W, spec.KH) == (EMBED, 512, 64, 1, 1)
    attn = kernels[_node(ir, "block.0.attn.core").id]
    assert isinstance(attn, SpikingSelfAttentionKernel)
    assert (attn.N, attn.C, attn.heads, attn.v_threshold) == (64, EMBED, HEADS, 0.5)
    assert attn.kv_numel == 8 * HEADS * (EMBED // HEADS) ** 2
    head = kernels[_node(ir, "head").id]
    assert isinstance(head, SpikeHeadKernel) and head.planes == 0 and head.HW == 64 and head.workspace_numel > 0
    assert _node(ir, "block.0.attn.k_linear").id not in kernels


def test_int_stream_rejects_unknown():
    p = random_params(3, embed=EMBED, depth=1, num_classes=10)
    ir = frontend.spikformer_ir(p, T=4, batch=2, in_hw=(32, 32), heads=HEADS)
    with pytest.raises(ValueError):
        passes.optimize_ir(ir, int_stream="bf16")
