"""Kernel-object contract: compile_all() -> {nid: kernel} (sengine/build/tilelang_compiler.py:404-491).

Kernel objects are cached per shape key (tilelang_compiler.py:551-553) and called the way
the reference runtime calls them (sengine/cuda_graph_runtime.py:616-643):

    spikes = kern(data, weight, state, bn_scale, bn_bias)   # fused node with a membrane
    spikes = kern(data, weight, bn_scale, bn_bias)          # no membrane: V0 = 0, not kept

`data` is the reference's fp16 NHWC (T*B, H, W, C_in) activation or an int32 spike-bit
tensor (T*B, H, W, C_in/32); the output uses the same encoding unless out_enc is given,
and is freshly allocated like a TileLang out_idx=[-1] result.  `weight` may be the
prepared SparseWeight blob (kern.prepare_weight) or the raw weight tensor in the
runtime's (KH, KW, C_in, C_out) layout (cuda_graph_runtime.py:233-235) or torch's
(C_out, C_in, KH, KW); raw tensors are compressed once and cached.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import torch

from . import ops
from .ops import ENC_BITS, ENC_F16, ConvSpec, SEngineError, tail_eligible

FUSED_VARIANTS = {"FusedSparseConvBNLIF", "TileLangFusedConvBNIF", "TileLangFusedConv1x1BNIF"}
DENSE_VARIANTS = {"TileLangConvBN", "TileLangConv1x1BN"}
NEURON_VARIANTS = {"CUDAVec4LIF", "CUDAVec4IF"}
STEM_VARIANTS = {"TileLangStemConvBN"}
HEAD_VARIANTS = {"CuBLASGemm"}
POOL_VARIANTS = {"CuDNNPool"}
ATTENTION_VARIANTS = {"FusedSpikformerAttn"}


class SparseWeight:
    """One contiguous device blob [2:4 values | position metadata] for a fused node: a single
    pointer carries both, which is what the 6-pointer call() ABI passes as `weight`."""

    def __init__(self, spec: ConvSpec, blob: torch.Tensor, value_bytes: int):
        self.spec = spec
        self.blob = blob
        self.value_bytes = value_bytes
        self.values = blob[:value_bytes].view(torch.int16)
        self.meta = blob[value_bytes:].view(torch.int32)

    def data_ptr(self) -> int:
        return self.blob.data_ptr()

    @classmethod
    def from_weight(cls, spec: ConvSpec, w: torch.Tensor, device=None, check_pattern=True,
                    tail=False) -> "SparseWeight":
        if isinstance(w, np.ndarray):
            w = torch.from_numpy(np.ascontiguousarray(w))
        device = device or (w.device if w.is_cuda else torch.device("cuda"))
        w = w.to(device).contiguous()
        layout = _weight_layout(spec, w)
        values, meta, _ = ops.compress_2_4(spec, w, layout, check_pattern=check_pattern, tail=tail)
        vb = values.numel() * 2
        blob = torch.empty(vb + meta.numel() * 4, dtype=torch.uint8, device=device)
        blob[:vb].copy_(values.view(torch.uint8))
        blob[vb:].copy_(meta.view(torch.uint8))
        return cls(spec, blob, vb)


def _cached_blob(cache: dict, w: torch.Tensor, prepare):
    """The prepared form of raw weight `w`, rebuilt when `w` is not the tensor (or a view of the
    storage) it was built from, or was modified in place since.  The cache keeps a reference to
    the tensor it was built from: while the entry lives, that memory cannot be freed and handed
    to a different weight (the caching allocator reuses addresses routinely), so equal
    (address, version, shape, strides, dtype) means the same bytes.  Views share their base's
    version counter, so an in-place update through any view is seen.  One entry per kernel
    object (the most recent weight)."""
    key = (w.data_ptr(), w._version, tuple(w.shape), tuple(w.stride()), w.dtype)
    hit = cache.get("entry")
    if hit is not None and hit[0] == key and hit[1].untyped_storage().data_ptr() == w.untyped_storage().data_ptr():
        return hit[2]
    blob = prepare(w)
    cache["entry"] = (key, w, blob)
    return blob


def _weight_layout(spec: ConvSpec, w: torch.Tensor) -> int:
    if tuple(w.shape) == (spec.C_out, spec.C_in, spec.KH, spec.KW):
        return ops.WLAYOUT_OIHW
    if tuple(w.shape) == (spec.KH, spec.KW, spec.C_in, spec.C_out):
        return ops.WLAYOUT_HWIO
    raise SEngineError(f"weight shape {tuple(w.shape)} matches neither OIHW nor HWIO for {spec}")


class FusedSparseConvBNLIFKernel:
    """The fused 2:4 Conv+BN+neuron node (one HIP launch per call).  in_planes > 1: the input
    is an integer activation stored as that many bit planes (spec.C_in counts plane
    channels); a raw weight of the conv's own C_in is expanded to planes here.  tail: the
    input's last 32 channels are zero padding and the node runs the paired-tail call (spike
    bits in and out, no traces)."""

    def __init__(self, spec: ConvSpec, key: str, in_planes: int = 1, tail: bool = False):
        self.spec = spec  # in_enc/out_enc of `spec` are ignored; chosen per call
        self.key = key
        self.in_planes = in_planes
        self.tail = tail
        self._wcache: dict = {}
        self.OH, self.OW, self.M, self.K_red = ops.geometry(spec)

    def spec_for(self, in_enc: int, out_enc: int) -> ConvSpec:
        return dataclasses.replace(self.spec, in_enc=in_enc, out_enc=out_enc)

    def prepare_weight(self, w, device=None) -> SparseWeight:
        if self.in_planes > 1 and not isinstance(w, SparseWeight):
            from .sparsity import expand_planes
            if isinstance(w, np.ndarray):
                w = torch.from_numpy(np.ascontiguousarray(w))
            if tuple(w.shape) == (self.spec.C_out, self.spec.C_in // self.in_planes, self.spec.KH, self.spec.KW):
                w = expand_planes(w.float(), self.in_planes)
        return SparseWeight.from_weight(self.spec, w, device, tail=self.tail)

    def _weight(self, w) -> SparseWeight:
        if isinstance(w, SparseWeight):
            return w
        if not isinstance(w, torch.Tensor):
            raise TypeError("weight must be a SparseWeight or a torch.Tensor")
        return _cached_blob(self._wcache, w, self.prepare_weight)

    def __call__(self, data: torch.Tensor, weight, *args, out_enc=None, out=None, h_trace=None, x_trace=None):
        if len(args) == 3:
            state, bn_scale, bn_bias = args
        elif len(args) == 2:
            state, (bn_scale, bn_bias) = None, args
        else:
            raise TypeError("call as kern(data, weight, state, bn_scale, bn_bias) or kern(data, weight, bn_scale, bn_bias)")
        in_enc = ENC_BITS if data.dtype == torch.int32 else ENC_F16 if data.dtype == torch.float16 else None
        if in_enc is None:
            raise SEngineError("data must be fp16 NHWC or int32 spike bits")
        spec = self.spec_for(in_enc, in_enc if out_enc is None else out_enc)
        sw = self._weight(weight)
        if self.tail:
            if h_trace is not None or x_trace is not None:
                raise SEngineError("a paired-tail node records no traces")
            return ops.fused_sparse_conv_bn_lif_tail(spec, data, sw.values, sw.meta, bn_scale, bn_bias, state=state,
                                                     out=out)
        return ops.fused_sparse_conv_bn_lif(spec, data, sw.values, sw.meta, bn_scale, bn_bias, state=state, out=out,
                                            h_trace=h_trace, x_trace=x_trace)


class StemConvBNKernel:
    """Dense fp32 stem conv + folded BN on the images (C_in = 3; TileLangStemConvBN), with the
    absorbed neuron over the T repeats and the spike max-pool in the same launch when given
    their buffers:  kern(x, weight, bn_scale, bn_bias, pooled=..., spikes=..., out=...)."""

    def __init__(self, spec: ConvSpec, key: str, pool=None):
        self.spec = spec
        self.key = key
        self.pool = pool  # (kernel, stride, pad) of the absorbed max-pool, or None

    def prepare_weight(self, w, device=None) -> torch.Tensor:
        if isinstance(w, np.ndarray):
            w = torch.from_numpy(np.ascontiguousarray(w))
        device = device or (w.device if w.is_cuda else torch.device("cuda"))
        w = w.to(device).float()
        if _weight_layout(self.spec, w) == ops.WLAYOUT_OIHW:
            w = w.permute(2, 3, 1, 0)
        return w.contiguous()  # HWIO: coalesced weight reads

    def __call__(self, x, weight, bn_scale, bn_bias, pooled=None, spikes=None, out=None):
        if pooled is not None:
            k, st, pd = self.pool
            return ops.stem_conv_bn_lif_pool(self.spec, x, weight, bn_scale, bn_bias, k, st, pd, pooled=pooled,
                                             spikes=spikes)[0]
        if spikes is not None:
            return ops.stem_conv_bn_neuron(self.spec, x, weight, bn_scale, bn_bias, out=out, spikes=spikes,
                                           want_out=out is not None)[1]
        return ops.stem_conv_bn(self.spec, x, weight, bn_scale, bn_bias, out=out, layout=ops.WLAYOUT_HWIO)


class SpikeHeadKernel:
    """GlobalAvgPool -> Flatten -> TemporalMean -> Gemm on (integer) spike activations
    (CuBLASGemm with the pool and mean absorbed): kern(x, fc_weight, fc_bias, out=..., workspace=...).
    planes 0: x is an integer-valued fp16 stream; a `workspace` of workspace_numel int32 then
    splits its sums over many workgroups per image."""

    def __init__(self, T: int, B: int, HW: int, C: int, planes: int, key: str):
        self.T, self.B, self.HW, self.C, self.planes, self.key = T, B, HW, C, planes, key

    @property
    def workspace_numel(self) -> int:
        return self.B * ops.HEAD_WS_SPLIT * self.C if self.planes == 0 else 0

    def __call__(self, x, fc_weight, fc_bias, out=None, workspace=None):
        return ops.sew_head(x, self.T, self.B, self.HW, self.C, self.planes, fc_weight, fc_bias, out=out,
                            workspace=workspace)


class SpikingSelfAttentionKernel:
    """The Spikformer attention core (FusedSpikformerAttn; sengine/tdl/attention_ops.py:48-98):
    kern(q, k, v, kv=..., out=...) on spike bits (T*B, N, C/32) -> the attention LIF's spike bits.
    kv: an int32 workspace of kv_numel elements (K^T V per head)."""

    def __init__(self, T: int, B: int, N: int, C: int, ap, key: str):
        self.T, self.B, self.N, self.C, self.key = T, B, N, C, key
        self.heads, self.scale = int(ap.num_heads), float(ap.scale)
        self.tau, self.v_threshold = float(ap.attn_lif_tau), float(ap.attn_lif_v_threshold)
        if self.heads * int(ap.head_dim) != C:
            raise SEngineError(f"attention: {self.heads} heads x {ap.head_dim} != {C} channels")

    @property
    def kv_numel(self) -> int:
        d = self.C // self.heads
        return self.T * self.B * self.heads * d * d

    def __call__(self, q, k, v, kv=None, out=None):
        return ops.spiking_self_attention(q, k, v, self.T, self.B, self.N, self.C, self.heads, scale=self.scale,
                                          neuron="lif", tau=self.tau, v_threshold=self.v_threshold, v_reset=0.0,
                                          kv=kv, out=out)


class DenseConvBNKernel:
    """Unfused fallback, Conv+BN half: kern(data, weight, bn_scale, bn_bias) -> fp32 (T*B, OH, OW, C_out)."""

    def __init__(self, spec: ConvSpec, key: str):
        self.spec = spec
        self.key = key
        self._wcache: dict = {}

    def prepare_weight(self, w, device=None) -> torch.Tensor:
        if isinstance(w, np.ndarray):
            w = torch.from_numpy(np.ascontiguousarray(w))
        device = device or (w.device if w.is_cuda else torch.device("cuda"))
        w = w.to(device).contiguous()
        return ops.pack_dense_weights(self.spec, w, _weight_layout(self.spec, w))

    def __call__(self, data: torch.Tensor, weight, bn_scale, bn_bias, out=None):
        in_enc = ENC_BITS if data.dtype == torch.int32 else ENC_F16 if data.dtype == torch.float16 else None
        if in_enc is None:
            raise SEngineError("data must be fp16 NHWC or int32 spike bits")
        spec = dataclasses.replace(self.spec, in_enc=in_enc)
        if isinstance(weight, torch.Tensor) and weight.dtype == torch.int16:
            blob = weight
        else:
            blob = _cached_blob(self._wcache, weight, self.prepare_weight)
        return ops.dense_conv_bn(spec, data, blob, bn_scale, bn_bias, out=out)


class RealConvBNKernel:
    """fp32 1x1 Conv + folded BN on a real-valued NHWC tensor (MS-ResNet's TDBN shortcut;
    TileLangConv1x1BN with a real input): kern(x, weight, bn_scale, bn_bias, in_T=..., out=...).
    in_T = 1: the input holds one timestep (a stem's output), every output is stored T times."""

    def __init__(self, spec: ConvSpec, key: str):
        self.spec = spec
        self.key = key

    def prepare_weight(self, w, device=None) -> torch.Tensor:
        if isinstance(w, np.ndarray):
            w = torch.from_numpy(np.ascontiguousarray(w))
        device = device or (w.device if w.is_cuda else torch.device("cuda"))
        w = w.to(device).float()
        if _weight_layout(self.spec, w) == ops.WLAYOUT_OIHW:
            w = w.permute(2, 3, 1, 0)
        return w.contiguous()  # HWIO (1, 1, C_in, C_out)

    def __call__(self, x, weight, bn_scale, bn_bias, in_T=None, out=None):
        return ops.real_conv_bn(self.spec, x, weight, bn_scale, bn_bias, in_T=in_T, out=out, layout=ops.WLAYOUT_HWIO)


class NeuronExt:
    """Standalone temporal neuron with the torch-extension API the reference JIT-builds
    (if_neuron / lif_neuron, sengine/csrc/green_context/if_neuron.cu:75-126):
    input (T*S, F) or any (T*spatial...) tensor, membrane with `spatial` elements; T =
    input.numel() / membrane.numel(); hard reset to 0; returns fp16 spikes shaped like input.
    The membrane is updated in place with the final state."""

    @staticmethod
    def _run(inp, membrane, v_threshold, neuron, tau):
        x = inp if inp.dtype == torch.float32 else inp.float()
        x = x.contiguous()
        n = membrane.numel()
        if x.numel() % n:
            raise SEngineError("input size must be a multiple of the membrane size")
        T = x.numel() // n
        s = ops.multistep_neuron(x, T, neuron, tau, v_threshold, 0.0, state=membrane, out_enc=ENC_F16)
        return s.view(inp.shape)

    def if_neuron(self, input, membrane, v_threshold=1.0):
        return self._run(input, membrane, v_threshold, "if", 1.0)

    def lif_neuron(self, input, membrane, v_threshold=1.0, recip_tau=0.5):
        return self._run(input, membrane, v_threshold, "lif", 1.0 / float(recip_tau))


_NEURON_EXT = NeuronExt()


def get_cuda_if() -> NeuronExt:
    """Name kept from tilelang_compiler.py (the neuron extension loader)."""
    return _NEURON_EXT


def _kname(node) -> str:
    kv = node.assigned_kernel
    return getattr(kv, "name", str(kv))


def _neuron_params(ir, node):
    ids = list(node.extra_attrs.get("absorbed_nids", [])) + list(ir.successors(node.id))
    for nid in ids:
        n = ir.nodes.get(nid)
        if n is not None and getattr(n, "neuron_params", None) is not None:
            return n.op_type.name, n.neuron_params
    return None, None


class SparseKernelCompiler:
    """compile_all() for the nodes this build serves; mirrors TileLangCompiler's contract.

    precision 'fp16': weights rounded to fp16 (one SMFMAC plane, the reference engine's
    io dtype); 'fp32': fp32-faithful weights as an fp16 hi + lo pair (two planes)."""

    def __init__(self, ir, batch_size: int = 1, precision: str = "fp16"):
        if precision not in ("fp16", "fp32"):
            raise ValueError("precision must be 'fp16' or 'fp32'")
        self.ir = ir
        self.T = int(getattr(ir, "T", 4) or 4)
        self.B = int(batch_size)
        self.precision = precision
        self._kernel_cache: dict = {}

    def _spec(self, node, neuron_kind, np_) -> ConvSpec:
        cp = node.conv_params
        N, C, H, W = node.input_shapes[0]
        if N != self.T * self.B:
            raise SEngineError(f"node {node.name}: input batch {N} != T*B = {self.T * self.B}")
        if cp.stride_h != cp.stride_w or cp.pad_h != cp.pad_w or cp.dilation_h != cp.dilation_w or cp.groups != 1:
            raise SEngineError(f"node {node.name}: only square stride/pad/dilation and groups=1 are supported")
        neuron = {"LIF": "lif", "IF": "if", "MS": "ms"}.get(neuron_kind, "if")
        hard = True if np_ is None else bool(np_.hard_reset)
        planes = int(node.extra_attrs.get("in_planes", 1))  # 0: an fp16 input
        c_out = int(node.extra_attrs.get("merged_out_channels", cp.out_channels))
        # LIF: tau; MS: the decay (models/msresnet.py:28-56; kept in tau, as NeuronParams does)
        return ConvSpec(T=self.T, B=self.B, C_in=cp.in_channels * max(planes, 1), H=H, W=W, C_out=c_out,
                        KH=cp.kernel_h, KW=cp.kernel_w, stride=cp.stride_h, padding=cp.pad_h,
                        dilation=cp.dilation_h, neuron=neuron, hard_reset=hard,
                        tau=float(np_.tau) if (np_ is not None and neuron != "if") else 2.0,
                        v_threshold=float(np_.v_threshold) if np_ is not None else 1.0,
                        v_reset=float(np_.v_reset) if np_ is not None else 0.0,
                        weight_planes=1 if self.precision == "fp16" else 2)

    def compile_all(self, skip_nids=None) -> dict:
        skip = skip_nids or set()
        kernels = {}
        for nid in self.ir.topo_order:
            if nid in skip:
                continue
            node = self.ir.nodes[nid]
            name = _kname(node)
            if name in FUSED_VARIANTS:
                if not node.sparse_weight:
                    raise SEngineError(f"node {node.name}: {name} needs 2:4 weights on this build "
                                       "(dense weights take the TileLangConvBN + neuron fallback)")
                kind, np_ = _neuron_params(self.ir, node)
                spec = self._spec(node, kind or "IF", np_)
                planes = int(node.extra_attrs.get("in_planes", 1))
                tail = planes == 1 and len(node.input_names) == 1 and \
                    tail_eligible(spec, node.extra_attrs.get("in_channels_real"))
                key = f"sparse_{spec}_{self.precision}" + ("_tail" if tail else "")
                kern = self._kernel_cache.get(key)
                if kern is None:
                    kern = FusedSparseConvBNLIFKernel(spec, key, planes, tail=tail)
                    self._kernel_cache[key] = kern
                node.tilelang_config = {"kernel": "fused_sparse_conv_bn_lif", "T": self.T, "waves": 4,
                                        "tile_channels": 64, "tile_positions": 64}
                kernels[nid] = kern
            elif name in DENSE_VARIANTS and node.extra_attrs.get("real_input"):
                spec = self._spec(node, "IF", None)
                key = f"real_{spec}"
                kern = self._kernel_cache.get(key)
                if kern is None:
                    kern = RealConvBNKernel(spec, key)
                    self._kernel_cache[key] = kern
                kernels[nid] = kern
            elif name in DENSE_VARIANTS:
                spec = self._spec(node, "IF", None)
                key = f"dense_{spec}_{self.precision}"
                kern = self._kernel_cache.get(key)
                if kern is None:
                    kern = DenseConvBNKernel(spec, key)
                    self._kernel_cache[key] = kern
                kernels[nid] = kern
            elif name in NEURON_VARIANTS:
                kernels[nid] = get_cuda_if()
            elif name in STEM_VARIANTS:
                kernels[nid] = self._stem(node)
            elif name in ATTENTION_VARIANTS:
                TB, C, H, W = node.input_shapes[0]
                ap = node.attention_params
                key = f"attn_{self.T}_{self.B}_{H * W}_{C}_{ap}"
                kern = self._kernel_cache.get(key)
                if kern is None:
                    kern = SpikingSelfAttentionKernel(self.T, self.B, H * W, C, ap, key)
                    self._kernel_cache[key] = kern
                kernels[nid] = kern
            elif name in HEAD_VARIANTS:
                first = self.ir.nodes[node.extra_attrs["absorbed_nids"][-1]]  # the chain's first op
                N, C, H, W = first.input_shapes[0]
                key = f"head_{self.T}_{self.B}_{H * W}_{C}_{node.extra_attrs.get('in_planes', 1)}"
                kernels[nid] = SpikeHeadKernel(self.T, self.B, H * W, C, int(node.extra_attrs.get("in_planes", 1)),
                                               key)
        return kernels

    def _stem(self, node):
        cp = node.conv_params
        N, C, H, W = node.input_shapes[0]
        if N != self.B:
            raise SEngineError(f"node {node.name}: stem input batch {N} != B = {self.B} (conv runs once per image)")
        if cp.stride_h != cp.stride_w or cp.pad_h != cp.pad_w or cp.groups != 1:
            raise SEngineError(f"node {node.name}: only square stride/pad and groups=1 are supported")
        neuron = self.ir.nodes[node.extra_attrs["neuron_nid"]]
        np_ = neuron.neuron_params
        kind = {"LIF": "lif", "IF": "if", "MS": "ms"}[neuron.op_type.name]
        spec = ConvSpec(T=self.T, B=self.B, C_in=C, H=H, W=W, C_out=cp.out_channels, KH=cp.kernel_h,
                        KW=cp.kernel_w, stride=cp.stride_h, padding=cp.pad_h, neuron=kind,
                        hard_reset=bool(np_.hard_reset), tau=float(np_.tau) if kind != "if" else 2.0,
                        v_threshold=float(np_.v_threshold), v_reset=float(np_.v_reset))
        pool = None
        for a in node.extra_attrs["absorbed_nids"]:
            pn = self.ir.nodes[a]
            if pn.op_type.name == "MaxPool":
                pp = pn.pool_params or {}
                pool = (int(pp.get("kernel_size", 3)), int(pp.get("stride", 2)), int(pp.get("padding", 1)))
        key = f"stem_{spec}_{pool}"
        kern = self._kernel_cache.get(key)
        if kern is None:
            kern = StemConvBNKernel(spec, key, pool)
            self._kernel_cache[key] = kern
        return kern
