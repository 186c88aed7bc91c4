"""Spikformer inference on the fused kernels, replayed as one hipGraph.

The reference model is models/spikformer.py: SPS patch splitting (:153-209), Blocks of
spiking self-attention and MLP with residual adds (:59-150), mean over tokens and T and a
Linear head (:273-288).  SpikformerEngine maps it onto this library:

* SPS: the first conv (C_in = 3, dense) runs once on the B images (the reference repeats the
  image over T before it, :283-285, so the T copies are equal), in the same launch as its
  LIF over the repeated output (sengine_amd_stem_conv_bn_neuron, the fp32 conv output not
  stored); the other four convs are fused 2:4 Conv+BN+LIF
  launches on spike bits, with spike max-pools after the third and fourth, and the
  relative-position conv's spikes added to the max-pooled features in its epilogue (an
  integer activation of 2 bit planes).  Channel counts that are not multiples of 64
  (embed/8 = 48, embed/4 = 96 for embed 384) are padded with zero weights and a zero BN
  affine: the padded channels never fire (V_th > 0) and multiply zero weights downstream;
* blocks: the token stream x (T*B, N tokens, embed) is integer-valued (the residual adds of
  spikes, :148-149).  stream="f16" (default) keeps it as fp16 integers, the reference's own
  representation: q, k, v and fc1 (Linear + BN1d + LIF, :103-125) are fused 1x1 convs over
  the token grid reading it as fp16 activations (K = embed), and proj / MLP fc2 write
  spike + x as fp16 in their epilogues.  stream="planes" stores it as bit planes instead:
  the token Linears then run on spike bits with plane-expanded weights (K = planes * embed)
  and the adds write planes.  The Linear bias is folded into the BN affine.  q, k and v read
  the same stream: their weights are concatenated along C_out (zero-padded to a multiple of
  256) and run as one launch whose spike bits are split into one plane per Linear
  (sengine_amd_fused_sparse_conv_bn_lif_split).  SSA runs as the two-kernel Q (K^T V) path
  with the attention LIF (V_th 0.5);
* head: mean over tokens and T of the integer stream and the Linear (sengine_amd_sew_head, or
  with the fp16 stream sengine_amd_sew_head_ws: the sums split over many workgroups).

Every buffer is allocated once; the launch sequence is captured into one hipGraph.
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass

import torch

from . import ops
from .ops import ConvSpec, SEngineError, tail_eligible
from .sparsity import expand_planes, fold_batchnorm, validate_2_4_pattern

ATTN_VTH = 0.5  # attn_lif threshold, models/spikformer.py:96


def _pad64(c: int) -> int:
    return (c + 63) // 64 * 64


def _planes(max_value: int) -> int:
    return max(1, int(max_value).bit_length())


def random_params(seed: int = 0, embed: int = 384, depth: int = 8, mlp_ratio: int = 4, num_classes: int = 1000,
                  in_channels: int = 3) -> dict:
    """Random Spikformer parameters with the reference's state_dict names and the model's own
    initialisation (models/spikformer.py:238-245: Linear weights N(0, 0.02) clamped to +-0.04,
    biases 0; Conv2d U(+-1/sqrt(fan_in)) and BatchNorm defaults), every conv after the first
    (C_in = 3) and every block Linear 2:4-pruned along its input and rounded to fp16
    (BASELINE config 4)."""
    import math
    from .sparsity import prune_conv_2_4
    g = torch.Generator().manual_seed(seed)
    p = {}

    def bn(name, c):
        p[name + ".weight"], p[name + ".bias"] = torch.ones(c), torch.zeros(c)
        p[name + ".running_mean"], p[name + ".running_var"] = torch.zeros(c), torch.ones(c)

    chans = [("proj_conv", in_channels, embed // 8), ("proj_conv1", embed // 8, embed // 4),
             ("proj_conv2", embed // 4, embed // 2), ("proj_conv3", embed // 2, embed), ("rpe_conv", embed, embed)]
    for name, cin, cout in chans:
        b = 1.0 / math.sqrt(cin * 9)
        w = (torch.rand((cout, cin, 3, 3), generator=g) * 2 - 1) * b
        p[f"patch_embed.{name}.weight"] = w if name == "proj_conv" else prune_conv_2_4(w).half().float()
        bn(f"patch_embed.{name.replace('conv', 'bn')}", cout)
    hidden = embed * mlp_ratio
    for i in range(depth):
        for lin, cin, cout in (("attn.q", embed, embed), ("attn.k", embed, embed), ("attn.v", embed, embed),
                               ("attn.proj", embed, embed), ("mlp.fc1", embed, hidden), ("mlp.fc2", hidden, embed)):
            w = (torch.randn((cout, cin, 1, 1), generator=g) * 0.02).clamp_(-0.04, 0.04)
            p[f"block.{i}.{lin}_linear.weight"] = prune_conv_2_4(w).half().float()[:, :, 0, 0]
            p[f"block.{i}.{lin}_linear.bias"] = torch.zeros(cout)
            bn(f"block.{i}.{lin}_bn", cout)
    p["head.weight"] = (torch.randn((num_classes, embed), generator=g) * 0.02).clamp_(-0.04, 0.04)
    p["head.bias"] = torch.zeros(num_classes)
    return p


@dataclass
class Fused:
    spec: ConvSpec
    values: torch.Tensor
    meta: torch.Tensor
    scale: torch.Tensor
    bias: torch.Tensor
    tail: bool = False  # the input's last 32 channels are zero padding: the paired-tail call


@dataclass
class SBlock:
    name: str
    planes_in: int
    planes_mid: int
    planes_out: int
    qkv: Fused  # attn.q, .k, .v concatenated: one launch, spikes split into one plane each
    proj: Fused
    fc1: Fused
    fc2: Fused
    bufs: dict


class SpikformerEngine:
    """Static-shape Spikformer forward for `batch` images of in_hw pixels (embed channels,
    `heads` heads, `depth` blocks, MLP ratio `mlp_ratio`)."""

    def __init__(self, params: dict, batch: int, T: int = 4, embed: int = 384, heads: int = 8, depth: int = 8,
                 mlp_ratio: int = 4, in_hw=(224, 224), in_channels: int = 3, device="cuda", stream: str = "f16"):
        if embed % 64 or embed % heads:
            raise SEngineError("embed must be a multiple of 64 and of heads")
        if stream not in ("f16", "planes"):
            raise SEngineError("stream must be 'f16' or 'planes'")
        self.stream = stream
        f16 = stream == "f16"
        H, W = in_hw
        if H % 4 or W % 4:
            raise SEngineError("image sides must be multiples of 4 (two stride-2 max-pools)")
        self.dev = torch.device(device)
        self.B, self.T, self.embed, self.heads, self.depth = batch, T, embed, heads, depth
        self.in_shape = (batch, in_channels, H, W)
        p = {k: v.detach().float().cpu() for k, v in params.items()}
        self.graph = None
        TB = T * batch
        i32 = dict(dtype=torch.int32, device=self.dev)

        # ---- SPS
        c8, c4, c2 = embed // 8, embed // 4, embed // 2
        P8, P4 = _pad64(c8), _pad64(c4)
        w0 = p["patch_embed.proj_conv.weight"]
        if tuple(w0.shape) != (c8, in_channels, 3, 3):
            raise SEngineError(f"patch_embed.proj_conv.weight: expected {(c8, in_channels, 3, 3)}")
        w0p = torch.zeros(P8, in_channels, 3, 3)
        w0p[:c8] = w0
        sc, bi = self._bn(p, "patch_embed.proj_bn", pad_to=P8)
        self.stem_spec = ConvSpec(T=1, B=batch, C_in=in_channels, H=H, W=W, C_out=P8, KH=3, KW=3, stride=1,
                                  padding=1)
        self.stem_w = w0p.permute(2, 3, 1, 0).contiguous().to(self.dev)  # HWIO
        self.stem_scale, self.stem_bias = sc.to(self.dev), bi.to(self.dev)
        self.x_buf = torch.zeros(self.in_shape, dtype=torch.float32, device=self.dev)
        # the stem's LIF over its output repeated T times runs in the stem launch; the fp32
        # output itself is not stored
        self.stem_nspec = dataclasses.replace(self.stem_spec, T=T, neuron="lif", hard_reset=True, tau=2.0,
                                              v_threshold=1.0, v_reset=0.0)
        self.s0 = torch.empty(TB, H, W, P8 // 32, **i32)
        self.c1 = self._conv(p, "proj_conv1", c8, c4, P8, P4, H, W)
        self.s1 = torch.empty(TB, H, W, P4 // 32, **i32)
        self.c2 = self._conv(p, "proj_conv2", c4, c2, P4, c2, H, W)
        self.s2 = torch.empty(TB, H, W, c2 // 32, **i32)
        self.H2, self.W2 = (H - 1) // 2 + 1, (W - 1) // 2 + 1
        self.p2 = torch.empty(TB, self.H2, self.W2, c2 // 32, **i32)
        self.c3 = self._conv(p, "proj_conv3", c2, embed, c2, embed, self.H2, self.W2)
        self.s3 = torch.empty(TB, self.H2, self.W2, embed // 32, **i32)
        self.H4, self.W4 = (self.H2 - 1) // 2 + 1, (self.W2 - 1) // 2 + 1
        self.p3 = torch.empty(TB, self.H4, self.W4, embed // 32, **i32)
        self.rpe = self._conv(p, "rpe_conv", embed, embed, embed, embed, self.H4, self.W4)
        self.N = self.H4 * self.W4
        maxv = 2  # rpe spike + max-pooled feature spike
        f16t = dict(dtype=torch.float16, device=self.dev)

        def stream_buf(planes):
            return torch.empty(TB, self.N, embed, **f16t) if f16 else torch.empty(TB, self.N, planes * embed // 32, **i32)

        self.x0 = stream_buf(_planes(maxv))
        if f16:  # rpe spikes + the pooled features (1 plane) written as fp16
            self.rpe = Fused(dataclasses.replace(self.rpe.spec, out_enc=ops.ENC_F16), self.rpe.values, self.rpe.meta,
                             self.rpe.scale, self.rpe.bias)

        # ---- blocks
        hidden = embed * mlp_ratio
        self.blocks: list[SBlock] = []
        for i in range(depth):
            pre = f"block.{i}"
            P0, P1, P2 = _planes(maxv), _planes(maxv + 1), _planes(maxv + 2)
            if f16:
                if maxv + 2 >= 2048:
                    raise SEngineError("the residual stream exceeds fp16's exact integers (depth too large)")
                P0 = P1 = P2 = 0
            elif P2 > 5:
                raise SEngineError("the residual stream needs more than 5 bit planes (depth too large)")
            blk = SBlock(pre, P0, P1, P2,
                         qkv=self._concat_qkv(p, pre, embed, P0),
                         proj=self._linear(p, pre + ".attn.proj", embed, embed, 1, out_f16=f16),
                         fc1=self._linear(p, pre + ".mlp.fc1", embed, hidden, P1),
                         fc2=self._linear(p, pre + ".mlp.fc2", hidden, embed, 1, out_f16=f16),
                         bufs={})
            d = embed // heads
            # q, k and v read the same stream: one launch over their concatenated weights, its
            # spike bits split into one plane per Linear (the fourth plane holds the padding)
            nplanes = -(-blk.qkv.spec.C_out // embed)
            blk.bufs["qkv"] = torch.empty(nplanes, TB, self.N, embed // 32, **i32)
            for j, n in enumerate(("q", "k", "v")):
                blk.bufs[n] = blk.bufs["qkv"][j]
            blk.bufs["a"] = torch.empty(TB, self.N, embed // 32, **i32)
            blk.bufs["kv"] = torch.empty(TB, heads, d, d, **i32)
            blk.bufs["x1"] = stream_buf(P1)
            blk.bufs["h"] = torch.empty(TB, self.N, hidden // 32, **i32)
            blk.bufs["x2"] = stream_buf(P2)
            self.blocks.append(blk)
            maxv += 2
        self.final_planes = 0 if f16 else (self.blocks[-1].planes_out if self.blocks else _planes(2))
        self.head_w = p["head.weight"].contiguous().to(self.dev)
        self.head_b = p["head.bias"].contiguous().to(self.dev)
        self.logits = torch.empty(batch, self.head_w.shape[0], dtype=torch.float32, device=self.dev)
        # the head's split per-channel sums of the fp16 stream (sengine_amd_sew_head_ws)
        self.head_ws = torch.empty(batch * ops.HEAD_WS_SPLIT * embed, dtype=torch.int32, device=self.dev)

    # ------------------------------------------------------------------ build helpers
    @staticmethod
    def _bn(p, name, conv_bias=None, pad_to=None):
        sc, bi = fold_batchnorm(p[name + ".weight"], p[name + ".bias"], p[name + ".running_mean"],
                                p[name + ".running_var"], 1e-5, conv_bias)
        if pad_to is not None and pad_to > sc.numel():  # padded channels: zero affine, never fire
            sc = torch.cat([sc, torch.zeros(pad_to - sc.numel())])
            bi = torch.cat([bi, torch.zeros(pad_to - bi.numel())])
        return sc, bi

    def _spec(self, cin, cout, k, h, w, pad) -> ConvSpec:
        return ConvSpec(T=self.T, B=self.B, C_in=cin, H=h, W=w, C_out=cout, KH=k, KW=k, stride=1, padding=pad,
                        neuron="lif", hard_reset=True, tau=2.0, v_threshold=1.0, v_reset=0.0)

    def _prepare(self, spec: ConvSpec, w4: torch.Tensor, sc, bi, tail: bool = False) -> Fused:
        values, meta, _ = ops.compress_2_4(spec, w4.contiguous().to(self.dev).half(), tail=tail)
        return Fused(spec, values, meta, sc.to(self.dev), bi.to(self.dev), tail)

    def _conv(self, p, name, cin, cout, cin_p, cout_p, h, w) -> Fused:
        wk = f"patch_embed.{name}.weight"
        w_ = p[wk]
        if tuple(w_.shape) != (cout, cin, 3, 3):
            raise SEngineError(f"{wk}: expected shape {(cout, cin, 3, 3)}, got {tuple(w_.shape)}")
        if not validate_2_4_pattern(w_):
            raise SEngineError(f"{wk}: not 2:4 sparse along C_in")
        wp = torch.zeros(cout_p, cin_p, 3, 3)
        wp[:cout, :cin] = w_
        sc, bi = self._bn(p, f"patch_embed.{name.replace('conv', 'bn')}", pad_to=cout_p)
        spec = self._spec(cin_p, cout_p, 3, h, w, 1)
        return self._prepare(spec, wp, sc, bi, tail=tail_eligible(spec, cin))

    def _concat_qkv(self, p, pre, cin, planes) -> Fused:
        """attn.q, .k and .v concatenated along C_out, padded with zero rows (and a zero BN
        affine: never fire) up to a multiple of 256 output channels, the persistent 1x1
        kernel's four-wave super-blocks."""
        parts = [self._linear_parts(p, f"{pre}.attn.{n}", cin, cin, planes) for n in ("q", "k", "v")]
        spec = parts[0][0]
        cp = -(-3 * cin // 256) * 256
        w = torch.zeros(cp, spec.C_in, 1, 1)
        w[:3 * cin] = torch.cat([wx for _, wx, _, _ in parts])
        zeros = torch.zeros(cp - 3 * cin)
        sc = torch.cat([s for _, _, s, _ in parts] + [zeros])
        bi = torch.cat([b for _, _, _, b in parts] + [zeros])
        return self._prepare(dataclasses.replace(spec, C_out=cp), w, sc, bi)

    def _linear(self, p, name, cin, cout, planes, out_f16=False) -> Fused:
        spec, wx, sc, bi = self._linear_parts(p, name, cin, cout, planes, out_f16)
        return self._prepare(spec, wx, sc, bi)

    def _linear_parts(self, p, name, cin, cout, planes, out_f16=False):
        """planes 0: fp16 input (the integer stream as fp16); 1: spike bits; > 1: bit planes
        (plane-expanded weights).  out_f16: the spike + residual add writes the fp16 stream."""
        wk = name + "_linear.weight"
        w_ = p[wk]
        if tuple(w_.shape) != (cout, cin):
            raise SEngineError(f"{wk}: expected shape {(cout, cin)}, got {tuple(w_.shape)}")
        w4 = w_[:, :, None, None]
        if not validate_2_4_pattern(w4):
            raise SEngineError(f"{wk}: not 2:4 sparse along its input")
        sc, bi = self._bn(p, name + "_bn", conv_bias=p[name + "_linear.bias"])
        wx = expand_planes(w4, planes) if planes > 1 else w4
        # tokens as a (T*B, N, 1) grid of pixels: a Linear is a 1x1 conv
        spec = self._spec(cin * max(planes, 1), cout, 1, self.N, 1, 0)
        if planes == 0:
            spec = dataclasses.replace(spec, in_enc=ops.ENC_F16)
        if out_f16:
            spec = dataclasses.replace(spec, out_enc=ops.ENC_F16)
        return spec, wx, sc, bi

    # ------------------------------------------------------------------ execution
    def _fused(self, f: Fused, data, out):
        if f.tail:
            ops.fused_sparse_conv_bn_lif_tail(f.spec, data.view(-1), f.values, f.meta, f.scale, f.bias, out=out)
        else:
            ops.fused_sparse_conv_bn_lif(f.spec, data.view(-1), f.values, f.meta, f.scale, f.bias, out=out)

    def _fused_add(self, f: Fused, data, residual, res_planes, out, out_planes):
        ops.fused_sparse_conv_bn_lif_add(f.spec, data.view(-1), f.values, f.meta, f.scale, f.bias, residual,
                                         res_planes, out_planes, out=out)

    def run_sps(self):
        ops.stem_conv_bn_neuron(self.stem_nspec, self.x_buf, self.stem_w, self.stem_scale, self.stem_bias,
                                want_out=False, spikes=self.s0)
        self._fused(self.c1, self.s0, self.s1)
        self._fused(self.c2, self.s1, self.s2)
        H, W = self.stem_spec.H, self.stem_spec.W
        TB = self.T * self.B
        ops.maxpool_spikes(self.s2, TB, H, W, self.embed // 2, 3, 2, 1, out=self.p2)
        self._fused(self.c3, self.p2, self.s3)
        ops.maxpool_spikes(self.s3, TB, self.H2, self.W2, self.embed, 3, 2, 1, out=self.p3)
        self._fused_add(self.rpe, self.p3, self.p3, 1, self.x0, _planes(2))

    def block_input(self, i: int):
        """(token stream, its planes; 0 = fp16) entering block i."""
        if i == 0:
            return self.x0, 0 if self.stream == "f16" else _planes(2)
        prev = self.blocks[i - 1]
        return prev.bufs["x2"], prev.planes_out

    def run_block(self, i: int, x: torch.Tensor | None = None):
        blk = self.blocks[i]
        if x is None:
            x, _ = self.block_input(i)
        b = blk.bufs
        qkv = blk.qkv
        ops.fused_sparse_conv_bn_lif_split(qkv.spec, x.view(-1), qkv.values, qkv.meta, qkv.scale, qkv.bias,
                                           self.embed, out=b["qkv"])
        ops.spiking_self_attention(b["q"], b["k"], b["v"], self.T, self.B, self.N, self.embed, self.heads,
                                   v_threshold=ATTN_VTH, kv=b["kv"], out=b["a"])
        self._fused_add(blk.proj, b["a"], x, blk.planes_in, b["x1"], blk.planes_mid)
        self._fused(blk.fc1, b["x1"], b["h"])
        self._fused_add(blk.fc2, b["h"], b["x1"], blk.planes_mid, b["x2"], blk.planes_out)

    def run_head(self):
        x, planes = self.block_input(len(self.blocks))
        ops.sew_head(x, self.T, self.B, self.N, self.embed, planes, self.head_w, self.head_b, out=self.logits,
                     workspace=self.head_ws if planes == 0 else None)

    def _run_all(self):
        self.run_sps()
        for i in range(len(self.blocks)):
            self.run_block(i)
        self.run_head()

    @property
    def launches(self) -> int:
        # SPS 7, 6 per block (q/k/v, SSA 2, proj, fc1, fc2), the head 1 (bit planes) or 2 (fp16
        # stream: split sums, then the head)
        return 7 + 6 * len(self.blocks) + (2 if self.block_input(len(self.blocks))[1] == 0 else 1)

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
