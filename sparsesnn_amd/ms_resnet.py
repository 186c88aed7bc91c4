"""MS-ResNet-18/34 inference on the fused kernels, replayed as one hipGraph.

The reference builds the network in models/msresnet.py (MSNeuron :28-56, TDBNContainer
:58-80, BasicBlock18 :87-112, MSResNet18 :119-161, ms_resnet34 :318-319).  Its blocks keep a
real-valued stream: a block's input x is the previous block's `out + shortcut`, the block
fires its own neuron on it (sn1), and the shortcut adds x (or a 1x1 TDBN conv of x) back
after conv_bn2.  MSResNetEngine maps that onto this library:

* stem + first block's sn1: dense fp32 conv 7x7/2 + folded BN on the B images and the neuron
  over that output repeated T times, one launch (sengine_amd_stem_conv_bn_neuron); the
  reference repeats the image over T before conv1 (:146-150), so the T copies are equal and
  the stem runs once, its fp32 output kept for block 0's shortcut;
* per block: conv_bn1 + sn2 as one fused 2:4 Conv+BN+neuron launch (spike bits in and out);
  conv_bn2 + BN + shortcut add as the membrane-shortcut epilogue
  (sengine_amd_fused_sparse_conv_bn_add_neuron), which stores the block output y (fp32, the
  next block's real-valued input) and fires the next neuron on it -- the next block's sn1,
  or sn_out after the last block -- so no separate add or neuron launch exists; where the
  stride or width changes, the shortcut is the fp32 1x1 conv + BN of sengine_amd_real_conv_bn
  on the real-valued block input (computed once and stored T times for the first block,
  whose input is the repeated stem output);
* head: mean over T, average pool and Linear of sn_out's spikes (sengine_amd_sew_head).

Weights are folded, 2:4-checked and compressed once; every buffer is allocated at build
time; the launch sequence is captured into one hipGraph.
"""
from __future__ import annotations

import dataclasses
import math
from dataclasses import dataclass

import torch

from . import ops
from .ops import ConvSpec, SEngineError
from .sparsity import fold_batchnorm, prune_conv_2_4, validate_2_4_pattern

DEPTHS = {18: (2, 2, 2, 2), 34: (3, 4, 6, 3)}
WIDTHS = (64, 128, 256, 512)
MS_DECAY, MS_THRESH = 0.25, 0.5  # MSNeuron defaults, models/msresnet.py:21-22


def block_names(depth: int = 34):
    """(state-dict prefix, C_in, C_out, stride, has_shortcut) of every block, forward order:
    the first block of every stage has stride 2 (models/msresnet.py:130-133,135-141)."""
    out, cin = [], 64
    for si, (planes, n) in enumerate(zip(WIDTHS, DEPTHS[depth])):
        for bi in range(n):
            s = 2 if bi == 0 else 1
            out.append((f"conv{si + 2}_x.{bi}", cin, planes, s, s != 1 or cin != planes))
            cin = planes
    return out


def random_params(seed: int = 0, depth: int = 34, num_classes: int = 1000, in_channels: int = 3) -> dict:
    """Random ms_resnet parameters with the reference's state_dict names and its default
    initialisation (Conv2d U(+-1/sqrt(fan_in)); BatchNorm3d weight 0.5 where the reference
    sets bn_init_thresh (conv1, conv_bn1, shortcut; models/msresnet.py:75-76), else 1; Linear
    U(+-1/sqrt(fan_in))), every conv but the stem 2:4-pruned by magnitude along C_in and
    rounded to fp16."""
    g = torch.Generator().manual_seed(seed)
    p = {}

    def conv(name, cin, cout, k, prune):
        b = 1.0 / math.sqrt(cin * k * k)
        w = (torch.rand((cout, cin, k, k), generator=g) * 2 - 1) * b
        p[name + ".weight"] = prune_conv_2_4(w).half().float() if prune else w

    def bn(name, c, thresh_init):
        p[name + ".weight"] = torch.full((c,), MS_THRESH if thresh_init else 1.0)
        p[name + ".bias"], p[name + ".running_mean"], p[name + ".running_var"] = \
            torch.zeros(c), torch.zeros(c), torch.ones(c)

    conv("conv1.module.0", in_channels, 64, 7, False)
    bn("conv1.module.1", 64, True)
    for pre, cin, cout, _, has_sc in block_names(depth):
        conv(pre + ".conv_bn1.module.0", cin, cout, 3, True)
        bn(pre + ".conv_bn1.module.1", cout, True)
        conv(pre + ".conv_bn2.module.0", cout, cout, 3, True)
        bn(pre + ".conv_bn2.module.1", cout, False)
        if has_sc:
            conv(pre + ".shortcut.module.0", cin, cout, 1, True)
            bn(pre + ".shortcut.module.1", cout, True)
    bound = 1.0 / math.sqrt(512)
    p["fc.weight"] = (torch.rand((num_classes, 512), generator=g) * 2 - 1) * bound
    p["fc.bias"] = (torch.rand(num_classes, generator=g) * 2 - 1) * bound
    return p


@dataclass
class MSConv:
    """A fused spike conv with its prepared weights."""
    spec: ConvSpec
    values: torch.Tensor
    meta: torch.Tensor
    scale: torch.Tensor
    bias: torch.Tensor


@dataclass
class MSBlock:
    name: str
    conv1: MSConv
    conv2: MSConv
    sc_spec: ConvSpec | None
    sc_w: torch.Tensor | None
    sc_scale: torch.Tensor | None
    sc_bias: torch.Tensor | None
    s1: torch.Tensor       # sn2 spikes (T*B, OH, OW, C/32)
    y: torch.Tensor        # block output, fp32 (T*B, OH, OW, C)
    spk: torch.Tensor      # next neuron's spikes on y (T*B, OH, OW, C/32)
    sc: torch.Tensor | None  # shortcut conv output, fp32


class MSResNetEngine:
    """Static-shape MS-ResNet forward for `batch` images of in_hw pixels.

    neuron: 'ms' (the reference's MSNeuron; tau = its decay, default 0.25, v_threshold
    default 0.5) or 'lif' (LIF, tau default 2, v_threshold default 1, hard reset to 0)."""

    def __init__(self, params: dict, batch: int, T: int = 4, depth: int = 34, neuron: str = "ms",
                 tau: float | None = None, v_threshold: float | None = None, in_hw=(224, 224), in_channels: int = 3,
                 device="cuda"):
        if neuron not in ("ms", "lif"):
            raise SEngineError("neuron must be 'ms' or 'lif'")
        if depth not in DEPTHS:
            raise SEngineError(f"depth must be one of {sorted(DEPTHS)}")
        self.dev = torch.device(device)
        self.B, self.T, self.depth, self.neuron = batch, T, depth, neuron
        self.tau = tau if tau is not None else (MS_DECAY if neuron == "ms" else 2.0)
        self.vth = v_threshold if v_threshold is not None else (MS_THRESH if neuron == "ms" else 1.0)
        H, W = in_hw
        self.in_shape = (batch, in_channels, H, W)
        p = {k: v.detach().float().cpu() for k, v in params.items()}
        self.graph = None

        sc, bi = self._bn(p, "conv1.module.1")
        self.stem_spec = ConvSpec(T=1, B=batch, C_in=in_channels, H=H, W=W, C_out=64, KH=7, KW=7, stride=2, padding=3)
        self.stem_w = p["conv1.module.0.weight"].permute(2, 3, 1, 0).contiguous().to(self.dev)  # HWIO
        self.stem_scale, self.stem_bias = sc.to(self.dev), bi.to(self.dev)
        h, w = (H + 6 - 7) // 2 + 1, (W + 6 - 7) // 2 + 1
        self.H1, self.W1 = h, w
        self.x_buf = torch.zeros(self.in_shape, dtype=torch.float32, device=self.dev)
        self.stem_out = torch.empty(batch, h, w, 64, dtype=torch.float32, device=self.dev)
        self.stem_spk = torch.empty(T * batch, h, w, 2, dtype=torch.int32, device=self.dev)
        # conv1 + the first block's sn1 over its output repeated T times, in one launch
        self.stem_nspec = dataclasses.replace(self.stem_spec, T=T, neuron=neuron, hard_reset=True, tau=self.tau,
                                              v_threshold=self.vth, v_reset=0.0)

        TB = T * batch
        self.blocks: list[MSBlock] = []
        for pre, cin, cout, s, has_sc in block_names(depth):
            oh, ow = (h + 2 - 3) // s + 1, (w + 2 - 3) // s + 1
            c1 = self._fused(p, pre + ".conv_bn1.module", cin, cout, s, h, w)
            c2 = self._fused(p, pre + ".conv_bn2.module", cout, cout, 1, oh, ow)
            sc_spec = sc_w = sc_s = sc_b = sc_buf = None
            if has_sc:
                wk = pre + ".shortcut.module.0.weight"
                w_ = p[wk]
                if tuple(w_.shape) != (cout, cin, 1, 1):
                    raise SEngineError(f"{wk}: expected shape {(cout, cin, 1, 1)}, got {tuple(w_.shape)}")
                sc_spec = ConvSpec(T=T, B=batch, C_in=cin, H=h, W=w, C_out=cout, KH=1, KW=1, stride=s, padding=0)
                sc_w = w_.reshape(cout, cin).t().contiguous().to(self.dev)  # HWIO (1, 1, C_in, C_out)
                sc_s, sc_b = self._bn(p, pre + ".shortcut.module.1")
                sc_s, sc_b = sc_s.to(self.dev), sc_b.to(self.dev)
                sc_buf = torch.empty(TB, oh, ow, cout, dtype=torch.float32, device=self.dev)
            blk = MSBlock(pre, c1, c2, sc_spec, sc_w, sc_s, sc_b,
                          s1=torch.empty(TB, oh, ow, cout // 32, dtype=torch.int32, device=self.dev),
                          y=torch.empty(TB, oh, ow, cout, dtype=torch.float32, device=self.dev),
                          spk=torch.empty(TB, oh, ow, cout // 32, dtype=torch.int32, device=self.dev),
                          sc=sc_buf)
            self.blocks.append(blk)
            h, w = oh, ow
        self.final_hw, self.final_c = h * w, WIDTHS[-1]
        self.fc_w = p["fc.weight"].contiguous().to(self.dev)
        self.fc_b = p["fc.bias"].contiguous().to(self.dev)
        self.logits = torch.empty(batch, self.fc_w.shape[0], dtype=torch.float32, device=self.dev)

    # ------------------------------------------------------------------ build helpers
    @staticmethod
    def _bn(p, name):
        return fold_batchnorm(p[name + ".weight"], p[name + ".bias"], p[name + ".running_mean"],
                              p[name + ".running_var"])

    def _spec(self, cin, cout, k, stride, pad, h, w) -> ConvSpec:
        return ConvSpec(T=self.T, B=self.B, C_in=cin, H=h, W=w, C_out=cout, KH=k, KW=k, stride=stride, padding=pad,
                        neuron=self.neuron, hard_reset=True, tau=self.tau, v_threshold=self.vth, v_reset=0.0)

    def _fused(self, p, prefix, cin, cout, stride, h, w) -> MSConv:
        wkey = prefix + ".0.weight"
        w_ = p[wkey]
        if tuple(w_.shape) != (cout, cin, 3, 3):
            raise SEngineError(f"{wkey}: expected shape {(cout, cin, 3, 3)}, got {tuple(w_.shape)}")
        if not validate_2_4_pattern(w_):
            raise SEngineError(f"{wkey}: not 2:4 sparse along C_in")
        sc, bi = self._bn(p, prefix + ".1")
        spec = self._spec(cin, cout, 3, stride, 1, h, w)
        values, meta, _ = ops.compress_2_4(spec, w_.contiguous().to(self.dev).half())
        return MSConv(spec, values, meta, sc.to(self.dev), bi.to(self.dev))

    # ------------------------------------------------------------------ execution
    def run_stem(self):
        ops.stem_conv_bn_neuron(self.stem_nspec, self.x_buf, self.stem_w, self.stem_scale, self.stem_bias,
                                out=self.stem_out, spikes=self.stem_spk)

    def block_input(self, i: int):
        """(real-valued input, its spikes, timesteps of the real input) of block i."""
        if i == 0:
            return self.stem_out, self.stem_spk, 1
        prev = self.blocks[i - 1]
        return prev.y, prev.spk, self.T

    def run_block(self, i: int, x_real: torch.Tensor | None = None, x_spk: torch.Tensor | None = None,
                  in_T: int | None = None):
        blk = self.blocks[i]
        if x_real is None:
            x_real, x_spk, in_T = self.block_input(i)
        c1, c2 = blk.conv1, blk.conv2
        ops.fused_sparse_conv_bn_lif(c1.spec, x_spk.view(-1), c1.values, c1.meta, c1.scale, c1.bias, out=blk.s1)
        if blk.sc_spec is not None:
            ops.real_conv_bn(blk.sc_spec, x_real, blk.sc_w, blk.sc_scale, blk.sc_bias, in_T=in_T, out=blk.sc,
                             layout=ops.WLAYOUT_HWIO)
            residual = blk.sc
        else:
            if in_T != self.T:
                raise SEngineError("an identity shortcut needs a T-step real-valued input")
            residual = x_real
        ops.fused_sparse_conv_bn_add_neuron(c2.spec, blk.s1.view(-1), c2.values, c2.meta, c2.scale, c2.bias,
                                            residual=residual, real_out=blk.y, out=blk.spk)

    def run_head(self):
        ops.sew_head(self.blocks[-1].spk, self.T, self.B, self.final_hw, self.final_c, 1, self.fc_w, self.fc_b,
                     out=self.logits)

    def _run_all(self):
        self.run_stem()
        for i in range(len(self.blocks)):
            self.run_block(i)
        self.run_head()

    @property
    def launches(self) -> int:
        return 1 + sum(3 if b.sc_spec is not None else 2 for b in self.blocks) + 1

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
