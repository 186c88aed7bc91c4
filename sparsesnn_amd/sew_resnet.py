"""SEW-ResNet-18 inference on the fused kernels, replayed as one hipGraph.

The reference builds this network in models/sewresnet.py (BasicBlock :27-66, SEWResNet
:123-210, sew_resnet18 :213-214) and runs it through its engine: parse -> fuse -> compile
-> plan buffers -> capture a CUDA graph (sengine/cuda_graph_runtime.py:28-198,538-760;
sengine/csrc/cpp_executor.cu:1270-1315).  SEWResNet18Engine does the same for one
MI355X from a parameter dict with the reference's state_dict key names:

* weights are folded (BN -> per-channel scale/bias, sengine/optimizer.py:126-191),
  2:4-checked and compressed once; convs whose input is an integer SEW sum take their
  input as bit planes with plane-expanded weights (sparsity.expand_planes);
* every activation buffer is allocated once at build time (a static plan: the network has
  no data-dependent shapes), so a forward is a fixed sequence of launches;
* that sequence is captured into a hipGraph (torch.cuda.CUDAGraph) and replayed.

Launch sequence: stem conv+BN (sengine_amd_stem_conv_bn), neuron on the stem output
repeated over T, spike max-pool, then per BasicBlock the fused conv1+BN+neuron, the fused
1x1 downsample where the shape changes, and the fused conv2+BN+neuron with the SEW
residual add in its epilogue, and finally the pooled/time-averaged Linear head.
"""
from __future__ import annotations

import dataclasses

from dataclasses import dataclass, field

import torch

from . import ops
from .ops import ConvSpec, SEngineError
from .sparsity import expand_planes, fold_batchnorm, validate_2_4_pattern

STAGES = ((64, 1), (128, 2), (256, 2), (512, 2))


def random_params(seed: int = 0, num_classes: int = 100, in_channels: int = 3, fp16_weights: bool = True) -> dict:
    """Randomly initialised sew_resnet18 parameters, as the reference initialises the model
    (models/sewresnet.py:155-160: conv kaiming_normal fan_out/relu, BN weight 1 / bias 0 with
    default running statistics, nn.Linear default uniform), with every conv except the stem
    2:4-pruned by magnitude along C_in, keyed by the reference's
    state_dict names.  fp16_weights rounds the pruned conv weights to fp16 (the kernels' A
    operand precision)."""
    import math
    from .sparsity import prune_conv_2_4
    g = torch.Generator().manual_seed(seed)
    p = {}

    def conv(name, cin, cout, k, prune=True):
        w = torch.randn((cout, cin, k, k), generator=g) * math.sqrt(2.0 / (cout * k * k))
        if prune:
            w = prune_conv_2_4(w)
            if fp16_weights:
                w = w.half().float()
        p[name + ".weight"] = w

    def bn(name, c):
        p[name + ".weight"], p[name + ".bias"] = torch.ones(c), torch.zeros(c)
        p[name + ".running_mean"], p[name + ".running_var"] = torch.zeros(c), torch.ones(c)

    conv("conv1", in_channels, 64, 7, prune=False)
    bn("bn1", 64)
    inplanes = 64
    for si, (planes, stride) in enumerate(STAGES):
        for bi in range(2):
            s = stride if bi == 0 else 1
            pre = f"layer{si + 1}.{bi}"
            conv(pre + ".conv1.module.0", inplanes, planes, 3)
            bn(pre + ".conv1.module.1", planes)
            conv(pre + ".conv2.module.0", planes, planes, 3)
            bn(pre + ".conv2.module.1", planes)
            if bi == 0 and (s != 1 or inplanes != planes):
                conv(pre + ".downsample.0.module.0", inplanes, planes, 1)
                bn(pre + ".downsample.0.module.1", planes)
            inplanes = planes
    bound = 1.0 / math.sqrt(512)
    p["fc.weight"] = (torch.rand((num_classes, 512), generator=g) * 2 - 1) * bound
    p["fc.bias"] = (torch.rand(num_classes, generator=g) * 2 - 1) * bound
    return p


def _planes_for(max_value: int) -> int:
    return max(1, int(max_value).bit_length())


@dataclass
class FusedConv:
    """One fused Conv+BN+neuron node with its prepared weights."""
    name: str
    spec: ConvSpec
    values: torch.Tensor
    meta: torch.Tensor
    scale: torch.Tensor
    bias: torch.Tensor
    in_planes: int


@dataclass
class Block:
    name: str
    conv1: FusedConv
    conv2: FusedConv
    downsample: FusedConv | None
    in_planes: int
    id_planes: int
    out_planes: int
    H: int
    W: int
    OH: int
    OW: int
    C_out: int
    stride: int
    bufs: dict = field(default_factory=dict)


class SEWResNet18Engine:
    """Static-shape SEW-ResNet-18 forward for `batch` images of in_hw pixels."""

    def __init__(self, params: dict, batch: int, T: int = 4, neuron: str = "lif", tau: float = 2.0,
                 v_threshold: float = 1.0, v_reset: float | None = 0.0, in_hw=(32, 32), in_channels: int = 3,
                 device="cuda", weight_precision: str = "fp16"):
        if neuron not in ("lif", "if"):
            raise SEngineError("neuron must be 'lif' or 'if'")
        self.dev = torch.device(device)
        self.B, self.T, self.neuron, self.tau, self.vth, self.vreset = batch, T, neuron, tau, v_threshold, v_reset
        self.planes_w = 1 if weight_precision == "fp16" else 2
        H, W = in_hw
        self.in_shape = (batch, in_channels, H, W)
        p = {k: v.detach().float().cpu() for k, v in params.items()}
        self.graph = None

        # ---- stem: dense fp32 conv 7x7/2 + BN, neuron over the repeated output, max-pool
        sc, bi = fold_batchnorm(p["bn1.weight"], p["bn1.bias"], p["bn1.running_mean"], p["bn1.running_var"])
        self.stem_spec = ConvSpec(T=1, B=batch, C_in=in_channels, H=H, W=W, C_out=64, KH=7, KW=7, stride=2, padding=3)
        self.stem_w = p["conv1.weight"].permute(2, 3, 1, 0).contiguous().to(self.dev)  # HWIO: coalesced
        self.stem_scale, self.stem_bias = sc.to(self.dev), bi.to(self.dev)
        self.H1, self.W1 = (H + 6 - 7) // 2 + 1, (W + 6 - 7) // 2 + 1
        self.H2, self.W2 = (self.H1 + 2 - 3) // 2 + 1, (self.W1 + 2 - 3) // 2 + 1
        self.x_buf = torch.zeros(self.in_shape, dtype=torch.float32, device=self.dev)
        self.stem_out = torch.empty(batch, self.H1, self.W1, 64, dtype=torch.float32, device=self.dev)
        self.stem_spk = torch.empty(T * batch, self.H1, self.W1, 2, dtype=torch.int32, device=self.dev)
        self.pool_out = torch.empty(T * batch, self.H2, self.W2, 2, dtype=torch.int32, device=self.dev)
        # stem + neuron + max-pool in one launch where one workgroup holds a whole image
        self.stem_nspec = dataclasses.replace(self.stem_spec, T=T, neuron=neuron, hard_reset=v_reset is not None,
                                              tau=tau, v_threshold=v_threshold,
                                              v_reset=0.0 if v_reset is None else v_reset)
        self.stem_fused = True
        try:
            self._run_stem_fused()
        except SEngineError:
            self.stem_fused = False

        # ---- blocks
        self.blocks: list[Block] = []
        inplanes, h, w = 64, self.H2, self.W2
        x_planes, x_max = 1, 1  # max-pool output is binary
        for si, (planes, stride) in enumerate(STAGES):
            for bi_ in range(2):
                s = stride if bi_ == 0 else 1
                pre = f"layer{si + 1}.{bi_}"
                oh, ow = (h + 2 - 3) // s + 1, (w + 2 - 3) // s + 1
                conv1 = self._fused(pre + ".conv1.module", p, inplanes, planes, 3, s, 1, h, w, x_planes)
                conv2 = self._fused(pre + ".conv2.module", p, planes, planes, 3, 1, 1, oh, ow, 1)
                ds = None
                if bi_ == 0 and (s != 1 or inplanes != planes):
                    ds = self._fused(pre + ".downsample.0.module", p, inplanes, planes, 1, s, 0, h, w, x_planes)
                    id_planes, id_max = 1, 1
                else:
                    id_planes, id_max = x_planes, x_max
                out_max = id_max + 1
                out_planes = _planes_for(out_max)
                if out_planes > 3:
                    raise SEngineError("SEW sums above 7 need more than 3 bit planes")
                blk = Block(pre, conv1, conv2, ds, x_planes, id_planes, out_planes, h, w, oh, ow, planes, s)
                TB = T * batch
                blk.bufs["s1"] = torch.empty(TB, oh, ow, planes // 32, dtype=torch.int32, device=self.dev)
                if ds is not None:
                    blk.bufs["ds"] = torch.empty(TB, oh, ow, planes // 32, dtype=torch.int32, device=self.dev)
                blk.bufs["out"] = torch.empty(TB, oh, ow, out_planes * planes // 32, dtype=torch.int32,
                                              device=self.dev)
                self.blocks.append(blk)
                inplanes, h, w, x_planes, x_max = planes, oh, ow, out_planes, out_max
        self.final_planes, self.final_hw, self.final_c = x_planes, h * w, inplanes
        self.fc_w = p["fc.weight"].contiguous().to(self.dev)
        self.fc_b = p["fc.bias"].contiguous().to(self.dev)
        self.logits = torch.empty(batch, self.fc_w.shape[0], dtype=torch.float32, device=self.dev)

    # ------------------------------------------------------------------ build helpers
    def _fused(self, prefix, p, cin, cout, k, stride, pad, h, w, in_planes) -> FusedConv:
        wkey = prefix + ".0.weight"
        bn = prefix + ".1"
        w_ = p[wkey]
        if tuple(w_.shape) != (cout, cin, k, k):
            raise SEngineError(f"{wkey}: expected shape {(cout, cin, k, k)}, got {tuple(w_.shape)}")
        if not validate_2_4_pattern(w_):
            raise SEngineError(f"{wkey}: not 2:4 sparse along C_in (prune it, or run it on the dense fallback)")
        sc, bi = fold_batchnorm(p[bn + ".weight"], p[bn + ".bias"], p[bn + ".running_mean"], p[bn + ".running_var"])
        wx = expand_planes(w_, in_planes) if in_planes > 1 else w_
        # (convs with <= 16 output pixels run in the library's flat small-output layout)
        geo = dict(C_in=cin * in_planes, H=h, W=w, KH=k, KW=k, stride=stride, padding=pad)
        spec = ConvSpec(T=self.T, B=self.B, C_out=cout, neuron=self.neuron, hard_reset=self.vreset is not None,
                        tau=self.tau, v_threshold=self.vth, v_reset=0.0 if self.vreset is None else self.vreset,
                        weight_planes=self.planes_w, **geo)
        wdev = wx.contiguous().to(self.dev)
        if self.planes_w == 1:
            wdev = wdev.half()
        values, meta, _ = ops.compress_2_4(spec, wdev)
        return FusedConv(prefix, spec, values, meta, sc.to(self.dev), bi.to(self.dev), in_planes)

    # ------------------------------------------------------------------ execution
    def _run_stem_fused(self):
        ops.stem_conv_bn_lif_pool(self.stem_nspec, self.x_buf, self.stem_w, self.stem_scale, self.stem_bias, 3, 2, 1,
                                  pooled=self.pool_out, spikes=self.stem_spk)

    def run_stem(self):
        if self.stem_fused:
            self._run_stem_fused()
            return
        ops.stem_conv_bn(self.stem_spec, self.x_buf, self.stem_w, self.stem_scale, self.stem_bias, out=self.stem_out,
                         layout=ops.WLAYOUT_HWIO)
        ops.multistep_neuron_repeat(self.stem_out, self.T, self.neuron, self.tau, self.vth, self.vreset,
                                    out=self.stem_spk.view(self.T, -1))
        ops.maxpool_spikes(self.stem_spk, self.T * self.B, self.H1, self.W1, 64, 3, 2, 1, out=self.pool_out)

    def block_input(self, i: int) -> torch.Tensor:
        return self.pool_out if i == 0 else self.blocks[i - 1].bufs["out"]

    def run_block(self, i: int, x: torch.Tensor | None = None):
        blk = self.blocks[i]
        x = self.block_input(i) if x is None else x
        c1, c2, ds = blk.conv1, blk.conv2, blk.downsample
        if ds is not None:
            # conv1 and the downsample read the same x: one launch for both
            ops.fused_sparse_conv_bn_lif_pair(c1.spec, ds.spec, x.view(-1), c1.values, c1.meta, c1.scale, c1.bias,
                                              ds.values, ds.meta, ds.scale, ds.bias, out0=blk.bufs["s1"],
                                              out1=blk.bufs["ds"])
            identity = blk.bufs["ds"]
        else:
            ops.fused_sparse_conv_bn_lif(c1.spec, x.view(-1), c1.values, c1.meta, c1.scale, c1.bias,
                                         out=blk.bufs["s1"])
            identity = x
        ops.fused_sparse_conv_bn_lif_add(c2.spec, blk.bufs["s1"].view(-1), c2.values, c2.meta, c2.scale, c2.bias,
                                         identity, blk.id_planes, blk.out_planes, out=blk.bufs["out"])

    def run_head(self):
        ops.sew_head(self.blocks[-1].bufs["out"], self.T, self.B, self.final_hw, self.final_c, self.final_planes,
                     self.fc_w, self.fc_b, out=self.logits)

    def _run_all(self):
        self.run_stem()
        for i in range(len(self.blocks)):
            self.run_block(i)
        self.run_head()

    @property
    def launches(self) -> int:
        """Kernel launches per forward: a block's conv1 and downsample share one launch when
        both run on the library's small-output kernel (fewer than 128 units of 64 positions
        x 64 channels)."""
        def small(spec):
            M = spec.B * ((spec.H + 2 * spec.padding - spec.KH) // spec.stride + 1) * \
                ((spec.W + 2 * spec.padding - spec.KW) // spec.stride + 1)
            return ((M + 63) // 64) * (spec.C_out // 64) < 128
        n = (1 if self.stem_fused else 3) + 1
        for blk in self.blocks:
            n += 2
            if blk.downsample is not None and not (small(blk.conv1.spec) and small(blk.downsample.spec)):
                n += 1
        return n

    def capture(self):
        """Capture the whole forward into a hipGraph (replayed by forward())."""
        s = torch.cuda.Stream(self.dev)
        s.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(s):
            self._run_all()  # warm-up on a side stream (no allocation happens in _run_all)
        torch.cuda.current_stream(self.dev).wait_stream(s)
        torch.cuda.synchronize(self.dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._run_all()
        self.graph = g
        return g

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Logits (B, num_classes) for images x (B, C, H, W) fp32; returns the engine's
        output buffer (overwritten by the next call)."""
        if tuple(x.shape) != self.in_shape:
            raise SEngineError(f"expected input {self.in_shape}, got {tuple(x.shape)}")
        self.x_buf.copy_(x)
        if self.graph is not None:
            self.graph.replay()
        else:
            self._run_all()
        return self.logits
