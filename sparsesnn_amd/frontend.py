"""Front ends: EngineIR straight from a SEW-ResNet, MS-ResNet or Spikformer module tree or state
dict (ONNX, the reference's route via sengine/parser.py:77-368, is not available to this build).

`sew_resnet_ir` walks the structure of the reference's `sew_resnet18` (models/sewresnet.py:
123-210): stem conv1 / bn1, the image repeated over T, sn1, maxpool, layer1..layer4 of
BasicBlocks (conv1 = SeqToANNContainer(conv3x3, BN) -> sn1, conv2 -> sn2, optional downsample =
Sequential(SeqToANNContainer(conv1x1, BN), neuron), out = sn2 + identity for connect_f 'ADD'),
avgpool, flatten, mean over T, fc.  It reads the weights through the module's state_dict() key
names (conv1.weight, layer1.0.conv1.module.0.weight, layer2.0.downsample.0.module.1.running_var,
fc.bias, ...), so a reference model object or its state dict both work.  The node kinds and
shapes (NCHW with N = T*B after the repeat) are those the reference's parser emits; the
passes in sparsesnn_amd/passes.py then fuse them.
"""
from __future__ import annotations

import numpy as np

from .ir import (AttentionParams, ConvParams, EngineIR, KernelVariant, Node, NeuronParams, NeuronType, OpType,
                 WeightInfo)

STAGES = ((64, 1), (128, 2), (256, 2), (512, 2))


def _state(model) -> dict:
    sd = model.state_dict() if hasattr(model, "state_dict") else model
    return {k: (v.detach().float().cpu().numpy() if hasattr(v, "detach") else np.asarray(v, np.float32))
            for k, v in sd.items()}


def _neuron_attrs(model, neuron, tau, v_threshold, v_reset):
    """Neuron kind and hyper-parameters of a module tree, else the arguments (a state dict
    carries neither).

    Kind: the model's `neuron_type` ("if" builds MultiStepIFNeuron, anything else
    MultiStepLIFNeuron, models/sewresnet.py:124,138), else the class name of its first neuron.
    Settings: the multi-step wrappers keep them on their single-step `neuron` member
    (MultiStepLIFNeuron.neuron = LIFNeuron(tau, v_threshold, v_reset), MultiStepIFNeuron.neuron =
    IFNeuron(v_threshold, v_reset), models/neurons.py:195-199,217-221); a module that holds them
    itself is read directly.  v_reset None means soft reset.  tau / v_threshold may be
    learnable parameters (0-d tensors)."""
    sn = getattr(model, "sn1", None)
    kind = getattr(model, "neuron_type", None)
    if kind is not None:
        neuron = "if" if str(kind).lower() == "if" else "lif"
    elif sn is not None:
        cls = type(sn).__name__.upper()
        if "LIF" in cls:
            neuron = "lif"
        elif "IF" in cls:
            neuron = "if"
    if sn is not None:
        core = getattr(sn, "neuron", sn)
        if neuron == "lif" and hasattr(core, "tau"):
            tau = float(core.tau)
        if hasattr(core, "v_threshold"):
            v_threshold = float(core.v_threshold)
        if hasattr(core, "v_reset"):
            v_reset = None if core.v_reset is None else float(core.v_reset)
    return neuron, tau, v_threshold, v_reset


class _Builder:
    def __init__(self, ir: EngineIR, sd: dict, T: int, neuron, tau, v_threshold, v_reset):
        self.ir, self.sd, self.T = ir, sd, T
        is_lif = neuron == "lif"
        self.op = OpType.LIF if is_lif else OpType.IF
        self.np = NeuronParams(NeuronType.LIF if is_lif else NeuronType.IF, T, float(tau) if is_lif else 1.0,
                               float(v_threshold), 0.0 if v_reset is None else float(v_reset), v_reset is not None)

    def add(self, node: Node) -> str:
        self.ir.add_node(node)
        return node.output_names[0]

    def conv(self, key, x, shape, stride, pad):
        w = self.sd[key + ".weight"]
        cout, cin, kh, kw = w.shape
        N, C, H, W = shape
        if C != cin:
            raise ValueError(f"{key}: input has {C} channels, weight expects {cin}")
        oh, ow = (H + 2 * pad - kh) // stride + 1, (W + 2 * pad - kw) // stride + 1
        self.ir.weights[key + ".weight"] = w
        out = (N, cout, oh, ow)
        return self.add(Node(0, key, OpType.Conv2d, input_names=[x], output_names=[key + ".out"],
                             input_shapes=[shape], output_shapes=[out],
                             conv_params=ConvParams(cin, cout, kh, kw, stride, stride, pad, pad),
                             weight_info=WeightInfo(key + ".weight", tuple(w.shape)))), out

    def bn(self, key, x, shape):
        names = {}
        for attr, suffix in (("bn_scale_name", "weight"), ("bn_bias_name", "bias"), ("bn_mean_name", "running_mean"),
                             ("bn_var_name", "running_var")):
            self.ir.weights[f"{key}.{suffix}"] = self.sd[f"{key}.{suffix}"]
            names[attr] = f"{key}.{suffix}"
        return self.add(Node(0, key, OpType.BatchNorm, input_names=[x], output_names=[key + ".out"],
                             input_shapes=[shape], output_shapes=[shape], extra_attrs=dict(names, epsilon=1e-5)))

    def neuron(self, name, x, shape):
        return self.add(Node(0, name, self.op, is_stateful=True, input_names=[x], output_names=[name + ".out"],
                             input_shapes=[shape], output_shapes=[shape], neuron_params=self.np))

    def simple(self, name, op, x, in_shape, out_shape, **kw):
        return self.add(Node(0, name, op, input_names=[x] if isinstance(x, str) else list(x),
                             output_names=[name + ".out"], input_shapes=[in_shape], output_shapes=[out_shape], **kw))


def sew_resnet_ir(model, T: int = 4, batch: int = 1, in_hw=(32, 32), neuron: str = "lif", tau: float = 2.0,
                  v_threshold: float = 1.0, v_reset=0.0, blocks=(2, 2, 2, 2), connect_f: str = "ADD") -> EngineIR:
    """EngineIR of a SEW-ResNet (BasicBlock, `blocks` per stage; (2, 2, 2, 2) = sew_resnet18)
    for `batch` images of in_hw pixels.  `model`: the module tree (its state_dict() is read,
    and connect_f / neuron parameters from its attributes when present) or a state dict with
    the same keys.  Only connect_f 'ADD' is served."""
    connect_f = getattr(model, "connect_f", connect_f)
    if connect_f != "ADD":
        raise ValueError(f"connect_f {connect_f!r}: only 'ADD' is served by the fused SEW epilogue")
    neuron, tau, v_threshold, v_reset = _neuron_attrs(model, neuron, tau, v_threshold, v_reset)
    sd = _state(model)
    ir = EngineIR()
    ir.T = T
    bld = _Builder(ir, sd, T, neuron, tau, v_threshold, v_reset)
    H, W = in_hw
    cin = sd["conv1.weight"].shape[1]

    # stem: conv1 + bn1 once per image, repeated over T, sn1, maxpool
    x, shp = bld.conv("conv1", "x", (batch, cin, H, W), 2, 3)
    x = bld.bn("bn1", x, shp)
    shp = (T * batch,) + shp[1:]
    x = bld.simple("sn1.repeat", OpType.Tile, x, (batch,) + shp[1:], shp, extra_attrs={"repeats": T})
    x = bld.neuron("sn1", x, shp)
    ph, pw = (shp[2] + 2 - 3) // 2 + 1, (shp[3] + 2 - 3) // 2 + 1
    pshape = shp[:2] + (ph, pw)
    x = bld.simple("maxpool", OpType.MaxPool, x, shp, pshape,
                   pool_params={"kernel_size": 3, "stride": 2, "padding": 1})
    shp = pshape

    inplanes = shp[1]
    for si, (planes, stride) in enumerate(STAGES[:len(blocks)]):
        for bi in range(blocks[si]):
            s = stride if bi == 0 else 1
            pre = f"layer{si + 1}.{bi}"
            a, ashp = bld.conv(pre + ".conv1.module.0", x, shp, s, 1)
            a = bld.bn(pre + ".conv1.module.1", a, ashp)
            a = bld.neuron(pre + ".sn1", a, ashp)
            b, bshp = bld.conv(pre + ".conv2.module.0", a, ashp, 1, 1)
            b = bld.bn(pre + ".conv2.module.1", b, bshp)
            b = bld.neuron(pre + ".sn2", b, bshp)
            identity = x
            if (pre + ".downsample.0.module.0.weight") in sd:
                d, dshp = bld.conv(pre + ".downsample.0.module.0", x, shp, s, 0)
                d = bld.bn(pre + ".downsample.0.module.1", d, dshp)
                identity = bld.neuron(pre + ".downsample.1", d, dshp)
            elif s != 1 or inplanes != planes:
                raise ValueError(f"{pre}: stride/width change without a downsample branch")
            x = bld.simple(pre + ".add", OpType.Add, [b, identity], bshp, bshp)
            shp, inplanes = bshp, planes

    # head: avgpool -> flatten -> mean over T -> fc
    N, C = shp[0], shp[1]
    x = bld.simple("avgpool", OpType.GlobalAvgPool, x, shp, (N, C, 1, 1))
    x = bld.simple("flatten", OpType.Flatten, x, (N, C, 1, 1), (N, C))
    x = bld.simple("mean", OpType.TemporalMean, x, (N, C), (batch, C))
    fw, fb = sd["fc.weight"], sd["fc.bias"]
    ir.weights["fc.weight"], ir.weights["fc.bias"] = fw, fb
    bld.add(Node(0, "fc", OpType.Gemm, input_names=[x], output_names=["logits"], input_shapes=[(batch, C)],
                 output_shapes=[(batch, fw.shape[0])], gemm_params={"transB": 1},
                 weight_info=WeightInfo("fc.weight", tuple(fw.shape)), bias_info=WeightInfo("fc.bias", tuple(fb.shape))))
    return ir


def ms_resnet_ir(model, T: int = 4, batch: int = 1, in_hw=(224, 224), depth: int = 34, neuron: str = "ms",
                 tau=None, v_threshold=None) -> EngineIR:
    """EngineIR of an MS-ResNet-18/34 (models/msresnet.py:87-161, 318-319) for `batch` images.

    Structure, as the reference's forward runs it: conv1 = TDBN(Conv2d 7x7/2, BN) on the image
    repeated over T (computed here once per image, then the Tile: the T copies are equal), then
    per block (BasicBlock18.forward): x -> sn1 -> conv_bn1 -> sn2 -> conv_bn2, plus the shortcut
    (a TDBN 1x1 conv of the real-valued x where the stride or width changes, else x itself),
    out = conv_bn2 + shortcut; after the last block sn_out, mean over T, average pool, fc.
    TDBNContainer's BatchNorm3d in eval mode is the same per-channel affine as BatchNorm2d.
    `model`: a module tree (its state_dict) or a state dict with the reference's key names
    (conv1.module.{0,1}, conv{2..5}_x.{i}.conv_bn{1,2}.module.{0,1}, ...shortcut.module.{0,1},
    fc).  neuron 'ms' builds the reference's MSNeuron (decay `tau`, default 0.25; threshold
    default 0.5) as OpType.MS; 'lif' a LIF (tau default 2, threshold 1, hard reset to 0)."""
    from .ms_resnet import MS_DECAY, MS_THRESH, block_names
    if neuron not in ("ms", "lif"):
        raise ValueError("neuron must be 'ms' or 'lif'")
    sd = _state(model)
    ir = EngineIR()
    ir.T = T
    is_ms = neuron == "ms"
    tau = float(tau if tau is not None else (MS_DECAY if is_ms else 2.0))
    vth = float(v_threshold if v_threshold is not None else (MS_THRESH if is_ms else 1.0))
    bld = _Builder(ir, sd, T, "lif", tau, vth, 0.0)
    if is_ms:
        bld.op = OpType.MS
        bld.np = NeuronParams(NeuronType.MS, T, tau, vth, 0.0, True)
    H, W = in_hw
    cin = sd["conv1.module.0.weight"].shape[1]

    # stem: conv + BN once per image, then the repeat over T
    x, shp = bld.conv("conv1.module.0", "x", (batch, cin, H, W), 2, 3)
    x = bld.bn("conv1.module.1", x, shp)
    shp = (T * batch,) + shp[1:]
    x = bld.simple("conv1.repeat", OpType.Tile, x, (batch,) + shp[1:], shp, extra_attrs={"repeats": T})

    for pre, _, cout, s, has_sc in block_names(depth):
        a = bld.neuron(pre + ".sn1", x, shp)
        a, ashp = bld.conv(pre + ".conv_bn1.module.0", a, shp, s, 1)
        a = bld.bn(pre + ".conv_bn1.module.1", a, ashp)
        a = bld.neuron(pre + ".sn2", a, ashp)
        b, bshp = bld.conv(pre + ".conv_bn2.module.0", a, ashp, 1, 1)
        b = bld.bn(pre + ".conv_bn2.module.1", b, bshp)
        sc = x
        if has_sc:
            if (pre + ".shortcut.module.0.weight") not in sd:
                raise ValueError(f"{pre}: stride/width change without a shortcut conv")
            sc, sshp = bld.conv(pre + ".shortcut.module.0", x, shp, s, 0)
            sc = bld.bn(pre + ".shortcut.module.1", sc, sshp)
        x = bld.simple(pre + ".add", OpType.Add, [b, sc], bshp, bshp)
        shp = bshp

    # head: sn_out, mean over T, average pool, flatten, fc
    x = bld.neuron("sn_out", x, shp)
    N, C, h, w = shp
    x = bld.simple("mean", OpType.TemporalMean, x, shp, (batch, C, h, w))
    x = bld.simple("avgpool", OpType.GlobalAvgPool, x, (batch, C, h, w), (batch, C, 1, 1))
    x = bld.simple("flatten", OpType.Flatten, x, (batch, C, 1, 1), (batch, C))
    fw, fb = sd["fc.weight"], sd["fc.bias"]
    ir.weights["fc.weight"], ir.weights["fc.bias"] = fw, fb
    bld.add(Node(0, "fc", OpType.Gemm, input_names=[x], output_names=["logits"], input_shapes=[(batch, C)],
                 output_shapes=[(batch, fw.shape[0])], gemm_params={"transB": 1},
                 weight_info=WeightInfo("fc.weight", tuple(fw.shape)), bias_info=WeightInfo("fc.bias", tuple(fb.shape))))
    return ir


def spikformer_ir(model, T: int = 4, batch: int = 1, in_hw=(224, 224), heads: int = 8, tau: float = 2.0,
                  v_threshold: float = 1.0, attn_v_threshold: float = 0.5) -> EngineIR:
    """EngineIR of a Spikformer (models/spikformer.py:153-288) for `batch` images of in_hw pixels.

    SPS (:153-209): proj_conv + proj_bn on the images, computed once per image (the forward
    repeats the image over T first, :283-285, so the T copies are equal), then the Tile and
    proj_lif; proj_conv1..3 + BN + LIF with a 3x3/2 max-pool after the third and fourth; the
    relative-position conv rpe_conv + rpe_bn + rpe_lif on the pooled features x_feat, added to
    them; the feature map viewed as T*B x N tokens (flatten(-2).transpose(-1, -2)).  Tokens are
    an (N, 1) grid here, NCHW (T*B, C, N, 1), which in the runtime's NHWC memory is the same
    bytes as the (H/4, W/4) feature map: the view is free, and every token Linear is a Linear
    node over that grid.  Blocks (:59-150): q, k, v = Linear + BatchNorm1d + LIF of x, the
    attention core as one FusedAttention node (the reference's FusedSpikformerAttention op,
    sengine/tdl/attention_ops.py:48-98: (Q K^T * 0.125) V per head, then attn_lif with
    V_th = attn_v_threshold), proj = Linear + BN + LIF, x1 = x + proj; fc1, fc2 = Linear + BN +
    LIF, x2 = x1 + fc2.  Head (:273-288): mean over the tokens, mean over T, Linear.

    `model`: a module tree (its state_dict; heads from block[0].attn.num_heads) or a state dict
    with the reference's key names (patch_embed.proj_conv, .proj_bn, .proj_conv1..3,
    .proj_bn1..3, .rpe_conv, .rpe_bn; block.{i}.attn.{q,k,v,proj}_{linear,bn};
    block.{i}.mlp.fc{1,2}_{linear,bn}; head).  Every neuron but attn_lif is a LIF with `tau`,
    `v_threshold` and hard reset to 0 (MultiStepLIFNeuron(tau=2.0), :26,93-104)."""
    blocks = getattr(model, "block", None)
    if blocks is not None and len(blocks) and hasattr(blocks[0], "attn"):
        heads = int(getattr(blocks[0].attn, "num_heads", heads))
    sd = _state(model)
    depth = 0
    while f"block.{depth}.attn.q_linear.weight" in sd:
        depth += 1
    ir = EngineIR()
    ir.T = T
    bld = _Builder(ir, sd, T, "lif", tau, v_threshold, 0.0)
    H, W = in_hw
    cin = sd["patch_embed.proj_conv.weight"].shape[1]
    pool = {"kernel_size": 3, "stride": 2, "padding": 1}

    def maxpool(name, x, shp):
        out = shp[:2] + ((shp[2] - 1) // 2 + 1, (shp[3] - 1) // 2 + 1)
        return bld.simple(name, OpType.MaxPool, x, shp, out, pool_params=dict(pool)), out

    def conv_bn_lif(idx, x, shp):
        x, shp = bld.conv(f"patch_embed.proj_conv{idx}", x, shp, 1, 1)
        x = bld.bn(f"patch_embed.proj_bn{idx}", x, shp)
        return bld.neuron(f"patch_embed.proj_lif{idx}", x, shp), shp

    # ---- SPS
    x, shp = bld.conv("patch_embed.proj_conv", "x", (batch, cin, H, W), 1, 1)
    x = bld.bn("patch_embed.proj_bn", x, shp)
    shp = (T * batch,) + shp[1:]
    x = bld.simple("patch_embed.repeat", OpType.Tile, x, (batch,) + shp[1:], shp, extra_attrs={"repeats": T})
    x = bld.neuron("patch_embed.proj_lif", x, shp)
    x, shp = conv_bn_lif(1, x, shp)
    x, shp = conv_bn_lif(2, x, shp)
    x, shp = maxpool("patch_embed.maxpool2", x, shp)
    x, shp = conv_bn_lif(3, x, shp)
    feat, shp = maxpool("patch_embed.maxpool3", x, shp)
    r, _ = bld.conv("patch_embed.rpe_conv", feat, shp, 1, 1)
    r = bld.bn("patch_embed.rpe_bn", r, shp)
    r = bld.neuron("patch_embed.rpe_lif", r, shp)
    x = bld.simple("patch_embed.add", OpType.Add, [r, feat], shp, shp)
    TB, C, h4, w4 = shp
    N = h4 * w4
    tok = (TB, C, N, 1)
    x = bld.simple("patch_embed.tokens", OpType.Reshape, x, shp, tok)
    if C % heads:
        raise ValueError(f"embed {C} is not a multiple of {heads} heads")

    def linear_bn_lif(pre, x, cin_, cout_, neuron=True):
        wk, bk = pre + "_linear.weight", pre + "_linear.bias"
        w = sd[wk]
        if tuple(w.shape) != (cout_, cin_):
            raise ValueError(f"{wk}: expected shape {(cout_, cin_)}, got {tuple(w.shape)}")
        ir.weights[wk] = w
        bias = None
        if bk in sd:
            ir.weights[bk] = sd[bk]
            bias = WeightInfo(bk, tuple(sd[bk].shape))
        oshp = (TB, cout_, N, 1)
        y = bld.add(Node(0, pre + "_linear", OpType.Linear, input_names=[x], output_names=[pre + "_linear.out"],
                         input_shapes=[(TB, cin_, N, 1)], output_shapes=[oshp], gemm_params={"N": cout_},
                         weight_info=WeightInfo(wk, tuple(w.shape)), bias_info=bias))
        y = bld.bn(pre + "_bn", y, oshp)
        return bld.neuron(pre + "_lif", y, oshp)

    # ---- blocks
    attn_np = NeuronParams(NeuronType.LIF, T, float(tau), float(attn_v_threshold), 0.0, True)
    for i in range(depth):
        pre = f"block.{i}"
        hidden = sd[f"{pre}.mlp.fc1_linear.weight"].shape[0]
        q, k, v = (linear_bn_lif(f"{pre}.attn.{n}", x, C, C) for n in ("q", "k", "v"))
        a = bld.add(Node(0, f"{pre}.attn.core", OpType.FusedAttention, is_stateful=True, input_names=[q, k, v],
                         output_names=[f"{pre}.attn.core.out"], input_shapes=[tok] * 3, output_shapes=[tok],
                         neuron_params=attn_np,
                         attention_params=AttentionParams("spikformer", heads, C // heads, 0.125, h4, w4,
                                                          float(tau), float(attn_v_threshold)),
                         assigned_kernel=KernelVariant.FusedSpikformerAttn))
        p_ = linear_bn_lif(f"{pre}.attn.proj", a, C, C)
        x = bld.simple(f"{pre}.add1", OpType.Add, [x, p_], tok, tok)
        f1 = linear_bn_lif(f"{pre}.mlp.fc1", x, C, hidden)
        f2 = linear_bn_lif(f"{pre}.mlp.fc2", f1, hidden, C)
        x = bld.simple(f"{pre}.add2", OpType.Add, [x, f2], tok, tok)

    # ---- head: mean over tokens, mean over T, Linear
    x = bld.simple("avgpool", OpType.GlobalAvgPool, x, tok, (TB, C, 1, 1))
    x = bld.simple("flatten", OpType.Flatten, x, (TB, C, 1, 1), (TB, C))
    x = bld.simple("mean", OpType.TemporalMean, x, (TB, C), (batch, C))
    fw, fb = sd["head.weight"], sd["head.bias"]
    ir.weights["head.weight"], ir.weights["head.bias"] = fw, fb
    bld.add(Node(0, "head", OpType.Gemm, input_names=[x], output_names=["logits"], input_shapes=[(batch, C)],
                 output_shapes=[(batch, fw.shape[0])], gemm_params={"transB": 1},
                 weight_info=WeightInfo("head.weight", tuple(fw.shape)),
                 bias_info=WeightInfo("head.bias", tuple(fb.shape))))
    return ir
