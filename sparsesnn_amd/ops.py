"""Torch-facing wrappers over the C ABI of libsengine_amd.so.

PyTorch is used for device memory and the current stream only; every op launches a
hand-written gfx950 HIP kernel and there is no fallback path.  Each wrapper checks the
tensors against the descriptor on the host before launching (the C ABI takes raw
pointers and cannot check buffer sizes itself).
"""
from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import (ENC_BITS, ENC_F16, ENC_F32, NEURON_IF, NEURON_LIF, NEURON_MS, WLAYOUT_HWIO, WLAYOUT_OIHW,
                   ConvLifDesc, SEngineError, check)

__all__ = [
    "ConvSpec", "make_desc", "geometry", "set_fused_kernel", "compress_2_4", "pack_dense_weights", "pack_spikes",
    "unpack_spikes", "fused_sparse_conv_bn_lif", "fused_sparse_conv_bn_lif_add", "stem_conv_bn",
    "multistep_neuron_repeat", "maxpool_spikes", "sew_head", "dense_conv_bn", "multistep_neuron", "SEngineError",
    "ENC_BITS", "ENC_F16", "ENC_F32", "NEURON_LIF", "NEURON_IF", "NEURON_MS", "WLAYOUT_OIHW", "WLAYOUT_HWIO",
    "neuron_code", "fused_sparse_conv_bn_add_neuron", "spiking_self_attention", "stem_conv_bn_neuron",
    "fused_sparse_conv_bn_lif_pair", "fused_sparse_conv_bn_lif_split", "fused_sparse_conv_bn_lif_tail", "tail_eligible",
    "fused_plan",
]


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_cuda(t: torch.Tensor, name: str):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise SEngineError(f"{name} must be on a HIP device (got {t.device})")
    if not t.is_contiguous():
        raise SEngineError(f"{name} must be contiguous")


def _require_numel(t: torch.Tensor, n: int, dtype, name: str):
    if t.dtype != dtype:
        raise SEngineError(f"{name}: expected dtype {dtype}, got {t.dtype}")
    if t.numel() != n:
        raise SEngineError(f"{name}: expected {n} elements, got {t.numel()}")


@dataclass(frozen=True)
class ConvSpec:
    """Shape + neuron parameters of one Conv+BN+neuron node (ConvParams + NeuronParams,
    sengine/ir.py:179-201, plus the T/B extents the reference bakes into each kernel)."""

    T: int
    B: int
    C_in: int
    H: int
    W: int
    C_out: int
    KH: int = 3
    KW: int = 3
    stride: int = 1
    padding: int = 1
    dilation: int = 1
    neuron: str = "lif"          # "lif" | "if" | "ms" (MS-ResNet neuron: `tau` holds its decay)
    hard_reset: bool = True
    tau: float = 2.0
    v_threshold: float = 1.0
    v_reset: float = 0.0
    in_enc: int = ENC_BITS
    out_enc: int = ENC_BITS
    weight_planes: int = 1

    def desc(self) -> ConvLifDesc:
        return make_desc(self)


_NEURON_CODES = {"lif": NEURON_LIF, "if": NEURON_IF, "ms": NEURON_MS}


def neuron_code(name: str) -> int:
    """C-ABI neuron kind for 'lif' | 'if' | 'ms'."""
    if name not in _NEURON_CODES:
        raise ValueError(f"neuron must be 'lif', 'if' or 'ms', got {name!r}")
    return _NEURON_CODES[name]


def make_desc(s: ConvSpec) -> ConvLifDesc:
    return ConvLifDesc(
        T=s.T, B=s.B, C_in=s.C_in, H=s.H, W=s.W, C_out=s.C_out, KH=s.KH, KW=s.KW,
        stride_h=s.stride, stride_w=s.stride, pad_h=s.padding, pad_w=s.padding,
        dil_h=s.dilation, dil_w=s.dilation,
        neuron=neuron_code(s.neuron), hard_reset=int(bool(s.hard_reset)),
        tau=float(s.tau), v_threshold=float(s.v_threshold), v_reset=float(s.v_reset),
        in_enc=s.in_enc, out_enc=s.out_enc, weight_planes=s.weight_planes)


def set_fused_kernel(choice: str) -> None:
    """Kernel for spike-bit inputs: 'auto' (split-K small-M kernel for small outputs, else the
    halo-tiled kernel where eligible, else the LDS-staged kernel), 'direct' (direct-gather
    kernel), 'lds' (LDS-staged kernel) or 'tile' (halo-tiled kernel where eligible)."""
    lib = _lib.load()
    check(lib.sengine_amd_set_fused_kernel({"auto": 0, "direct": 1, "lds": 2, "tile": 3}[choice]),
          "set_fused_kernel")


PLAN_TRACES, PLAN_STATE, PLAN_SEW_ADD, PLAN_SHORTCUT, PLAN_TAIL = 1, 2, 4, 8, 16


def fused_plan(s: ConvSpec, traces: bool = False, state: bool = False, sew_add: bool = False,
               shortcut: bool = False, tail: bool = False) -> str:
    """Name of the kernel instance a fused call with these optional buffers would launch
    (route and compile-time specialisation); tail: the paired-tail call
    (fused_sparse_conv_bn_lif_tail).  Host-only, launches nothing."""
    lib = _lib.load()
    d = make_desc(s)
    flags = ((PLAN_TRACES if traces else 0) | (PLAN_STATE if state else 0) | (PLAN_SEW_ADD if sew_add else 0)
             | (PLAN_SHORTCUT if shortcut else 0) | (PLAN_TAIL if tail else 0))
    buf = ctypes.create_string_buffer(256)
    check(lib.sengine_amd_fused_plan(ctypes.byref(d), flags, buf, len(buf)), "fused_plan")
    return buf.value.decode()


def geometry(s: ConvSpec):
    """(OH, OW, M_per_t, K_red) of a node."""
    lib = _lib.load()
    d = make_desc(s)
    oh, ow = ctypes.c_int32(), ctypes.c_int32()
    m, k = ctypes.c_int64(), ctypes.c_int64()
    check(lib.sengine_amd_conv_geometry(ctypes.byref(d), ctypes.byref(oh), ctypes.byref(ow),
                                        ctypes.byref(m), ctypes.byref(k)), "conv_geometry")
    return oh.value, ow.value, m.value, k.value


def _enc_numel(enc: int, n_values: int) -> tuple:
    """(dtype, numel) of a tensor holding n_values activations in encoding enc."""
    if enc == ENC_BITS:
        if n_values % 32:
            raise SEngineError("bit-encoded tensors need a multiple of 32 values")
        return torch.int32, n_values // 32
    if enc == ENC_F16:
        return torch.float16, n_values
    if enc == ENC_F32:
        return torch.float32, n_values
    raise SEngineError(f"unknown encoding {enc}")


def _weight_enc(w: torch.Tensor) -> int:
    if w.dtype == torch.float32:
        return ENC_F32
    if w.dtype == torch.float16:
        return ENC_F16
    raise SEngineError(f"weights must be fp32 or fp16, got {w.dtype}")


def _check_weight(s: ConvSpec, w: torch.Tensor, layout: int):
    _require_cuda(w, "weight")
    shape = (s.C_out, s.C_in, s.KH, s.KW) if layout == WLAYOUT_OIHW else (s.KH, s.KW, s.C_in, s.C_out)
    if tuple(w.shape) != shape:
        raise SEngineError(f"weight: expected shape {shape}, got {tuple(w.shape)}")


def _blob_bytes(lib, d, tail: bool):
    vb, mb = ctypes.c_size_t(), ctypes.c_size_t()
    if tail:
        check(lib.sengine_amd_tail_blob_bytes(ctypes.byref(d), ctypes.byref(vb), ctypes.byref(mb)), "tail_blob_bytes")
    else:
        check(lib.sengine_amd_sparse_blob_bytes(ctypes.byref(d), ctypes.byref(vb), ctypes.byref(mb)),
              "sparse_blob_bytes")
    return vb, mb


def compress_2_4(s: ConvSpec, weight: torch.Tensor, layout: int = WLAYOUT_OIHW, check_pattern: bool = True,
                 tail: bool = False):
    """2:4-compress a conv weight on the GPU -> (values int16 tensor, meta int32 tensor, violations).

    Raises if check_pattern and any 4-group along C_in holds more than two entries with
    |w| >= 1e-10 (such weights belong on the dense fallback, sengine/optimizer.py:845-853).
    tail: the blob of the paired-tail call (fused_sparse_conv_bn_lif_tail), for a 3x3 conv
    whose last 32 input channels are zero padding; a nonzero weight there is a violation."""
    lib = _lib.load()
    _check_weight(s, weight, layout)
    d = make_desc(s)
    vb, mb = _blob_bytes(lib, d, tail)
    dev = weight.device
    values = torch.empty(vb.value // 2, dtype=torch.int16, device=dev)
    meta = torch.empty(mb.value // 4, dtype=torch.int32, device=dev)
    n_groups = lib.sengine_amd_num_groups(ctypes.byref(d))
    # zeroed: in the flat (small-output) layout taps that never touch the image are not visited
    viol = torch.zeros(n_groups, dtype=torch.int32, device=dev)
    fn = lib.sengine_amd_compress_2_4_tail if tail else lib.sengine_amd_compress_2_4
    check(fn(ctypes.byref(d), _ptr(weight), _weight_enc(weight), layout, _ptr(values), _ptr(meta), _ptr(viol),
             _stream(dev)), "compress_2_4")
    if check_pattern:
        n_bad = int(viol.sum().item())
        if n_bad:
            raise SEngineError(f"compress_2_4: {n_bad} 4-groups have more than two non-zero weights"
                               + (" or a nonzero weight in the last 32 (padding) input channels" if tail else ""))
    return values, meta, viol


def pack_dense_weights(s: ConvSpec, weight: torch.Tensor, layout: int = WLAYOUT_OIHW) -> torch.Tensor:
    lib = _lib.load()
    _check_weight(s, weight, layout)
    d = make_desc(s)
    vb = ctypes.c_size_t()
    check(lib.sengine_amd_dense_blob_bytes(ctypes.byref(d), ctypes.byref(vb)), "dense_blob_bytes")
    values = torch.empty(vb.value // 2, dtype=torch.int16, device=weight.device)
    check(lib.sengine_amd_pack_dense_weights(ctypes.byref(d), _ptr(weight), _weight_enc(weight), layout,
                                             _ptr(values), _stream(weight.device)), "pack_dense_weights")
    return values


def pack_spikes(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Dense (..., C) fp16/fp32 -> spike bits int32 (..., C/32) (value != 0 -> 1)."""
    lib = _lib.load()
    _require_cuda(x, "x")
    C = x.shape[-1]
    if C % 32:
        raise SEngineError("pack_spikes: last dim must be a multiple of 32")
    enc = ENC_F16 if x.dtype == torch.float16 else ENC_F32 if x.dtype == torch.float32 else None
    if enc is None:
        raise SEngineError("pack_spikes: x must be fp16 or fp32")
    n_pos = x.numel() // C
    if out is None:
        out = torch.empty(*x.shape[:-1], C // 32, dtype=torch.int32, device=x.device)
    else:
        _require_cuda(out, "out")
        _require_numel(out, n_pos * (C // 32), torch.int32, "out")
    check(lib.sengine_amd_pack_spikes(_ptr(x), enc, n_pos, C, _ptr(out), _stream(x.device)), "pack_spikes")
    return out


def unpack_spikes(bits: torch.Tensor, C: int, dtype=torch.float16, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    lib = _lib.load()
    _require_cuda(bits, "bits")
    if C % 32 or bits.shape[-1] != C // 32 or bits.dtype != torch.int32:
        raise SEngineError("unpack_spikes: bits must be int32 (..., C/32)")
    enc = ENC_F16 if dtype == torch.float16 else ENC_F32 if dtype == torch.float32 else None
    if enc is None:
        raise SEngineError("unpack_spikes: dtype must be fp16 or fp32")
    n_pos = bits.numel() // (C // 32)
    if out is None:
        out = torch.empty(*bits.shape[:-1], C, dtype=dtype, device=bits.device)
    else:
        _require_cuda(out, "out")
        _require_numel(out, n_pos * C, dtype, "out")
    check(lib.sengine_amd_unpack_spikes(_ptr(bits), n_pos, C, _ptr(out), enc, _stream(bits.device)), "unpack_spikes")
    return out


def fused_sparse_conv_bn_lif(s: ConvSpec, data: torch.Tensor, values: torch.Tensor, meta: torch.Tensor,
                             bn_scale: torch.Tensor, bn_bias: torch.Tensor, state: Optional[torch.Tensor] = None,
                             out: Optional[torch.Tensor] = None, h_trace: Optional[torch.Tensor] = None,
                             x_trace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused 2:4 Conv + BN + multi-step neuron (one launch).  Returns the spike tensor:
    bits int32 (T*B, OH, OW, C_out/32) or fp16 (T*B, OH, OW, C_out) per s.out_enc."""
    lib = _lib.load()
    OH, OW, M, _ = geometry(s)
    d = make_desc(s)
    vb, mb = ctypes.c_size_t(), ctypes.c_size_t()
    check(lib.sengine_amd_sparse_blob_bytes(ctypes.byref(d), ctypes.byref(vb), ctypes.byref(mb)), "sparse_blob_bytes")
    for t, n in ((data, "data"), (values, "values"), (meta, "meta"), (bn_scale, "bn_scale"), (bn_bias, "bn_bias")):
        _require_cuda(t, n)
    dev = data.device
    dt, n_in = _enc_numel(s.in_enc, s.T * s.B * s.H * s.W * s.C_in)
    _require_numel(data, n_in, dt, "data")
    if values.numel() * values.element_size() != vb.value or meta.numel() * meta.element_size() != mb.value:
        raise SEngineError("fused_sparse_conv_bn_lif: weight blob does not match the descriptor")
    _require_numel(bn_scale, s.C_out, torch.float32, "bn_scale")
    _require_numel(bn_bias, s.C_out, torch.float32, "bn_bias")
    if state is not None:
        _require_cuda(state, "state")
        _require_numel(state, M * s.C_out, torch.float32, "state")
    for tr, n in ((h_trace, "h_trace"), (x_trace, "x_trace")):
        if tr is not None:
            _require_cuda(tr, n)
            _require_numel(tr, s.T * M * s.C_out, torch.float32, n)
    odt, n_out = _enc_numel(s.out_enc, s.T * M * s.C_out)
    if out is None:
        last = s.C_out // 32 if s.out_enc == ENC_BITS else s.C_out
        out = torch.empty(s.T * s.B, OH, OW, last, dtype=odt, device=dev)
    else:
        _require_cuda(out, "out")
        _require_numel(out, n_out, odt, "out")
    rc = lib.sengine_amd_fused_sparse_conv_bn_lif(
        ctypes.byref(d), _ptr(data), _ptr(values), _ptr(meta), _ptr(state), _ptr(bn_scale), _ptr(bn_bias),
        _ptr(out), _ptr(h_trace), _ptr(x_trace), _stream(dev))
    check(rc, "fused_sparse_conv_bn_lif")
    return out


def tail_eligible(spec: ConvSpec, in_channels_real) -> bool:
    """Whether a fused 3x3 node whose last 32 input channels are zero padding runs the paired-tail
    call (fused_sparse_conv_bn_lif_tail: the last chunk's 32 real channels of two taps per
    reduction step) -- opt-in, SENGINE_AMD_TAIL=1 (read when an engine is built), where the
    shape and neuron allow it: it does 22 % fewer SMFMACs but runs on the persistent 3x3 kernel,
    which measured slower on such multi-chunk layers than the ordinary call over the padded
    blob (Spikformer's proj_conv2: 1,234-1,248 us against 1,192)."""
    return (os.environ.get("SENGINE_AMD_TAIL", "0") == "1" and in_channels_real is not None and int(in_channels_real) == spec.C_in - 32 and spec.KH == 3
            and spec.KW == 3 and spec.stride == 1 and spec.padding == 1 and spec.dilation == 1 and spec.T == 4
            and spec.weight_planes == 1 and spec.hard_reset and spec.v_reset == 0.0
            and (spec.neuron == "if" or (spec.neuron == "lif" and math.log2(spec.tau).is_integer())))


def fused_sparse_conv_bn_lif_tail(s: ConvSpec, data: torch.Tensor, values: torch.Tensor, meta: torch.Tensor,
                                  bn_scale: torch.Tensor, bn_bias: torch.Tensor, state: Optional[torch.Tensor] = None,
                                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The paired-tail fused call: a 3x3 conv whose last 32 input channels are zero padding, with
    the blob of compress_2_4(..., tail=True); spike bits in and out, T = 4, no traces.  Returns
    the spike bits int32 (T*B, OH, OW, C_out/32)."""
    lib = _lib.load()
    OH, OW, M, _ = geometry(s)
    d = make_desc(s)
    vb, mb = _blob_bytes(lib, d, True)
    for t, n in ((data, "data"), (values, "values"), (meta, "meta"), (bn_scale, "bn_scale"), (bn_bias, "bn_bias")):
        _require_cuda(t, n)
    dt, n_in = _enc_numel(s.in_enc, s.T * s.B * s.H * s.W * s.C_in)
    _require_numel(data, n_in, dt, "data")
    if values.numel() * values.element_size() != vb.value or meta.numel() * meta.element_size() != mb.value:
        raise SEngineError("fused_sparse_conv_bn_lif_tail: weight blob does not match the descriptor")
    _require_numel(bn_scale, s.C_out, torch.float32, "bn_scale")
    _require_numel(bn_bias, s.C_out, torch.float32, "bn_bias")
    if state is not None:
        _require_cuda(state, "state")
        _require_numel(state, M * s.C_out, torch.float32, "state")
    odt, n_out = _enc_numel(s.out_enc, s.T * M * s.C_out)
    if out is None:
        out = torch.empty(s.T * s.B, OH, OW, s.C_out // 32, dtype=odt, device=data.device)
    else:
        _require_cuda(out, "out")
        _require_numel(out, n_out, odt, "out")
    check(lib.sengine_amd_fused_sparse_conv_bn_lif_tail(ctypes.byref(d), _ptr(data), _ptr(values), _ptr(meta),
                                                        _ptr(state), _ptr(bn_scale), _ptr(bn_bias), _ptr(out),
                                                        _stream(data.device)), "fused_sparse_conv_bn_lif_tail")
    return out


def fused_sparse_conv_bn_lif_split(s: ConvSpec, data: torch.Tensor, values: torch.Tensor, meta: torch.Tensor,
                                   bn_scale: torch.Tensor, bn_bias: torch.Tensor, split: int,
                                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fused_sparse_conv_bn_lif with the spike bits split by channel into planes of `split`
    channels (layers concatenated along C_out that read the same input): returns int32
    (ceil(C_out / split), T*B, OH, OW, split/32); plane k holds channels [k*split, (k+1)*split)."""
    lib = _lib.load()
    if s.out_enc != ENC_BITS:
        raise SEngineError("fused_sparse_conv_bn_lif_split: spike-bit output only")
    OH, OW, M, _ = geometry(s)
    d = make_desc(s)
    vb, mb = ctypes.c_size_t(), ctypes.c_size_t()
    check(lib.sengine_amd_sparse_blob_bytes(ctypes.byref(d), ctypes.byref(vb), ctypes.byref(mb)), "sparse_blob_bytes")
    for t, n in ((data, "data"), (values, "values"), (meta, "meta"), (bn_scale, "bn_scale"), (bn_bias, "bn_bias")):
        _require_cuda(t, n)
    dt, n_in = _enc_numel(s.in_enc, s.T * s.B * s.H * s.W * s.C_in)
    _require_numel(data, n_in, dt, "data")
    if values.numel() * values.element_size() != vb.value or meta.numel() * meta.element_size() != mb.value:
        raise SEngineError("fused_sparse_conv_bn_lif_split: weight blob does not match the descriptor")
    _require_numel(bn_scale, s.C_out, torch.float32, "bn_scale")
    _require_numel(bn_bias, s.C_out, torch.float32, "bn_bias")
    nplanes = -(-s.C_out // split)
    if out is None:
        out = torch.empty(nplanes, s.T * s.B, OH, OW, split // 32, dtype=torch.int32, device=data.device)
    else:
        _require_cuda(out, "out")
        _require_numel(out, nplanes * s.T * M * split // 32, torch.int32, "out")
    check(lib.sengine_amd_fused_sparse_conv_bn_lif_split(
        ctypes.byref(d), _ptr(data), _ptr(values), _ptr(meta), None, _ptr(bn_scale), _ptr(bn_bias), _ptr(out), split,
        _stream(data.device)), "fused_sparse_conv_bn_lif_split")
    return out


def fused_sparse_conv_bn_lif_pair(s0: ConvSpec, s1: ConvSpec, data: torch.Tensor, values0: torch.Tensor,
                                  meta0: torch.Tensor, bn_scale0: torch.Tensor, bn_bias0: torch.Tensor,
                                  values1: torch.Tensor, meta1: torch.Tensor, bn_scale1: torch.Tensor,
                                  bn_bias1: torch.Tensor, out0: Optional[torch.Tensor] = None,
                                  out1: Optional[torch.Tensor] = None):
    """Two fused 2:4 Conv + BN + neuron nodes on the same input (a block's conv1 and its
    downsample), one launch where both run on the small-output kernel.  Returns (out0, out1),
    each as fused_sparse_conv_bn_lif would."""
    lib = _lib.load()
    for s in (s0, s1):
        if (s.T, s.B, s.C_in, s.H, s.W, s.in_enc) != (s0.T, s0.B, s0.C_in, s0.H, s0.W, s0.in_enc):
            raise SEngineError("fused_sparse_conv_bn_lif_pair: the two convs must read the same input")
    dev = data.device
    dt, n_in = _enc_numel(s0.in_enc, s0.T * s0.B * s0.H * s0.W * s0.C_in)
    _require_cuda(data, "data")
    _require_numel(data, n_in, dt, "data")
    outs = []
    for s, values, meta, sc, bi, out, tag in ((s0, values0, meta0, bn_scale0, bn_bias0, out0, "0"),
                                               (s1, values1, meta1, bn_scale1, bn_bias1, out1, "1")):
        OH, OW, M, _ = geometry(s)
        d = make_desc(s)
        vb, mb = ctypes.c_size_t(), ctypes.c_size_t()
        check(lib.sengine_amd_sparse_blob_bytes(ctypes.byref(d), ctypes.byref(vb), ctypes.byref(mb)),
              "sparse_blob_bytes")
        for t, n in ((values, "values"), (meta, "meta"), (sc, "bn_scale"), (bi, "bn_bias")):
            _require_cuda(t, n + tag)
        if values.numel() * values.element_size() != vb.value or meta.numel() * meta.element_size() != mb.value:
            raise SEngineError(f"fused_sparse_conv_bn_lif_pair: weight blob {tag} does not match its descriptor")
        _require_numel(sc, s.C_out, torch.float32, "bn_scale" + tag)
        _require_numel(bi, s.C_out, torch.float32, "bn_bias" + tag)
        odt, n_out = _enc_numel(s.out_enc, s.T * M * s.C_out)
        if out is None:
            last = s.C_out // 32 if s.out_enc == ENC_BITS else s.C_out
            out = torch.empty(s.T * s.B, OH, OW, last, dtype=odt, device=dev)
        else:
            _require_cuda(out, "out" + tag)
            _require_numel(out, n_out, odt, "out" + tag)
        outs.append(out)
    d0, d1 = make_desc(s0), make_desc(s1)
    check(lib.sengine_amd_fused_sparse_conv_bn_lif_pair(
        ctypes.byref(d0), ctypes.byref(d1), _ptr(data), _ptr(values0), _ptr(meta0), _ptr(bn_scale0), _ptr(bn_bias0),
        _ptr(outs[0]), _ptr(values1), _ptr(meta1), _ptr(bn_scale1), _ptr(bn_bias1), _ptr(outs[1]), _stream(dev)),
        "fused_sparse_conv_bn_lif_pair")
    return outs[0], outs[1]


def fused_sparse_conv_bn_lif_add(s: ConvSpec, data: torch.Tensor, values: torch.Tensor, meta: torch.Tensor,
                                 bn_scale: torch.Tensor, bn_bias: torch.Tensor, residual: torch.Tensor,
                                 residual_planes: int, out_planes: int, state: Optional[torch.Tensor] = None,
                                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused 2:4 Conv + BN + neuron + SEW 'ADD' residual: out = spike + residual as
    `out_planes` bit planes, int32 (T*B, OH, OW, out_planes*C_out/32).  With s.out_enc ==
    ENC_F16, out is fp16 (T*B, OH, OW, C_out) and the residual fp16 of that shape
    (residual_planes == 0) or `residual_planes` bit planes; out_planes is unused."""
    lib = _lib.load()
    f16 = s.out_enc == ENC_F16
    if s.out_enc != ENC_BITS and not f16:
        raise SEngineError("fused_sparse_conv_bn_lif_add: out_enc must be ENC_BITS or ENC_F16")
    OH, OW, M, _ = geometry(s)
    d = make_desc(s)
    vb, mb = ctypes.c_size_t(), ctypes.c_size_t()
    check(lib.sengine_amd_sparse_blob_bytes(ctypes.byref(d), ctypes.byref(vb), ctypes.byref(mb)), "sparse_blob_bytes")
    for t, n in ((data, "data"), (values, "values"), (meta, "meta"), (bn_scale, "bn_scale"), (bn_bias, "bn_bias"),
                 (residual, "residual")):
        _require_cuda(t, n)
    dev = data.device
    dt, n_in = _enc_numel(s.in_enc, s.T * s.B * s.H * s.W * s.C_in)
    _require_numel(data, n_in, dt, "data")
    if values.numel() * values.element_size() != vb.value or meta.numel() * meta.element_size() != mb.value:
        raise SEngineError("fused_sparse_conv_bn_lif_add: weight blob does not match the descriptor")
    _require_numel(bn_scale, s.C_out, torch.float32, "bn_scale")
    _require_numel(bn_bias, s.C_out, torch.float32, "bn_bias")
    if f16 and residual_planes == 0:
        out_planes = 0
        _require_numel(residual, s.T * M * s.C_out, torch.float16, "residual")
    else:
        _require_numel(residual, s.T * M * residual_planes * s.C_out // 32, torch.int32, "residual")
    if state is not None:
        _require_cuda(state, "state")
        _require_numel(state, M * s.C_out, torch.float32, "state")
    if out is None:
        out = (torch.empty(s.T * s.B, OH, OW, s.C_out, dtype=torch.float16, device=dev) if f16 else
               torch.empty(s.T * s.B, OH, OW, out_planes * s.C_out // 32, dtype=torch.int32, device=dev))
    else:
        _require_cuda(out, "out")
        if f16:
            _require_numel(out, s.T * M * s.C_out, torch.float16, "out")
        else:
            _require_numel(out, s.T * M * out_planes * s.C_out // 32, torch.int32, "out")
    rc = lib.sengine_amd_fused_sparse_conv_bn_lif_add(
        ctypes.byref(d), _ptr(data), _ptr(values), _ptr(meta), _ptr(state), _ptr(bn_scale), _ptr(bn_bias),
        _ptr(residual), int(residual_planes), _ptr(out), int(out_planes), _stream(dev))
    check(rc, "fused_sparse_conv_bn_lif_add")
    return out


def fused_sparse_conv_bn_add_neuron(s: ConvSpec, data: torch.Tensor, values: torch.Tensor, meta: torch.Tensor,
                                    bn_scale: torch.Tensor, bn_bias: torch.Tensor,
                                    residual: Optional[torch.Tensor] = None, state: Optional[torch.Tensor] = None,
                                    real_out: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
    """Membrane-shortcut form (MS-ResNet): y = BN(conv(data)) + residual (fp32 NHWC
    (T*B, OH, OW, C_out), or none) and the neuron of `s` run over y.  Returns (y, spikes)."""
    lib = _lib.load()
    OH, OW, M, _ = geometry(s)
    d = make_desc(s)
    vb, mb = ctypes.c_size_t(), ctypes.c_size_t()
    check(lib.sengine_amd_sparse_blob_bytes(ctypes.byref(d), ctypes.byref(vb), ctypes.byref(mb)), "sparse_blob_bytes")
    for t, n in ((data, "data"), (values, "values"), (meta, "meta"), (bn_scale, "bn_scale"), (bn_bias, "bn_bias")):
        _require_cuda(t, n)
    dev = data.device
    dt, n_in = _enc_numel(s.in_enc, s.T * s.B * s.H * s.W * s.C_in)
    _require_numel(data, n_in, dt, "data")
    if values.numel() * values.element_size() != vb.value or meta.numel() * meta.element_size() != mb.value:
        raise SEngineError("fused_sparse_conv_bn_add_neuron: weight blob does not match the descriptor")
    _require_numel(bn_scale, s.C_out, torch.float32, "bn_scale")
    _require_numel(bn_bias, s.C_out, torch.float32, "bn_bias")
    n_real = s.T * M * s.C_out
    if residual is not None:
        _require_cuda(residual, "residual")
        _require_numel(residual, n_real, torch.float32, "residual")
    if state is not None:
        _require_cuda(state, "state")
        _require_numel(state, M * s.C_out, torch.float32, "state")
    if real_out is None:
        real_out = torch.empty(s.T * s.B, OH, OW, s.C_out, dtype=torch.float32, device=dev)
    else:
        _require_cuda(real_out, "real_out")
        _require_numel(real_out, n_real, torch.float32, "real_out")
    odt, n_out = _enc_numel(s.out_enc, s.T * M * s.C_out)
    if out is None:
        last = s.C_out // 32 if s.out_enc == ENC_BITS else s.C_out
        out = torch.empty(s.T * s.B, OH, OW, last, dtype=odt, device=dev)
    else:
        _require_cuda(out, "out")
        _require_numel(out, n_out, odt, "out")
    rc = lib.sengine_amd_fused_sparse_conv_bn_add_neuron(
        ctypes.byref(d), _ptr(data), _ptr(values), _ptr(meta), _ptr(state), _ptr(bn_scale), _ptr(bn_bias),
        _ptr(residual), _ptr(real_out), _ptr(out), _stream(dev))
    check(rc, "fused_sparse_conv_bn_add_neuron")
    return real_out, out


def real_conv_bn(s: ConvSpec, x: torch.Tensor, weight: torch.Tensor, bn_scale: torch.Tensor, bn_bias: torch.Tensor,
                 in_T: Optional[int] = None, out: Optional[torch.Tensor] = None,
                 layout: int = WLAYOUT_OIHW) -> torch.Tensor:
    """MS-ResNet shortcut: fp32 1x1 conv (stride s.stride) + folded BN on the real-valued
    NHWC input x (in_T*s.B, H, W, C_in) -> fp32 NHWC (s.T*s.B, OH, OW, C_out).  in_T = 1
    (one timestep of input, e.g. the stem output) stores every output value s.T times;
    default in_T = s.T.  weight: OIHW (C_out, C_in, 1, 1) or HWIO (1, 1, C_in, C_out)."""
    lib = _lib.load()
    in_T = s.T if in_T is None else in_T
    for t, n in ((x, "x"), (weight, "weight"), (bn_scale, "bn_scale"), (bn_bias, "bn_bias")):
        _require_cuda(t, n)
    _require_numel(x, in_T * s.B * s.H * s.W * s.C_in, torch.float32, "x")
    _require_numel(weight, s.C_out * s.C_in, torch.float32, "weight")
    _require_numel(bn_scale, s.C_out, torch.float32, "bn_scale")
    _require_numel(bn_bias, s.C_out, torch.float32, "bn_bias")
    OH, OW = (s.H - 1) // s.stride + 1, (s.W - 1) // s.stride + 1
    if out is None:
        out = torch.empty(s.T * s.B, OH, OW, s.C_out, dtype=torch.float32, device=x.device)
    else:
        _require_cuda(out, "out")
        _require_numel(out, s.T * s.B * OH * OW * s.C_out, torch.float32, "out")
    d = make_desc(s)
    check(lib.sengine_amd_real_conv_bn(ctypes.byref(d), _ptr(x), int(in_T), _ptr(weight), int(layout),
                                       _ptr(bn_scale), _ptr(bn_bias), _ptr(out), _stream(x.device)), "real_conv_bn")
    return out


def spiking_self_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, T: int, B: int, N: int, C: int,
                           heads: int, scale: float = 0.125, neuron: str = "lif", tau: float = 2.0,
                           v_threshold: float = 0.5, v_reset: Optional[float] = 0.0,
                           kv: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Spikformer SSA on spike bits: q, k, v int32 (T*B, N, C/32) -> the attention neuron's
    spikes over T of (Q K^T * scale) V per head, int32 (T*B, N, C/32).  kv: optional
    workspace int32 (T*B, heads, d, d) (K^T V per head)."""
    lib = _lib.load()
    n_bits = T * B * N * C // 32
    for t, name in ((q, "q"), (k, "k"), (v, "v")):
        _require_cuda(t, name)
        _require_numel(t, n_bits, torch.int32, name)
    d = C // heads if heads else 0
    if kv is None:
        kv = torch.empty(T * B, heads, d, d, dtype=torch.int32, device=q.device)
    else:
        _require_cuda(kv, "kv")
        _require_numel(kv, T * B * heads * d * d, torch.int32, "kv")
    if out is None:
        out = torch.empty(T * B, N, C // 32, dtype=torch.int32, device=q.device)
    else:
        _require_cuda(out, "out")
        _require_numel(out, n_bits, torch.int32, "out")
    st = _stream(q.device)
    check(lib.sengine_amd_ssa_kv(T, B, N, C, heads, _ptr(k), _ptr(v), _ptr(kv), st), "ssa_kv")
    hard = v_reset is not None
    check(lib.sengine_amd_ssa_attend_neuron(T, B, N, C, heads, float(scale), neuron_code(neuron), int(hard),
                                            float(tau), float(v_threshold), float(v_reset if hard else 0.0),
                                            _ptr(q), _ptr(kv), _ptr(out), st), "ssa_attend_neuron")
    return out


def stem_conv_bn(s: ConvSpec, x: torch.Tensor, weight: torch.Tensor, bn_scale: torch.Tensor, bn_bias: torch.Tensor,
                 out: Optional[torch.Tensor] = None, layout: int = WLAYOUT_OIHW) -> torch.Tensor:
    """Dense fp32 conv + folded BN on NCHW images (s.B images; s.T ignored) -> NHWC fp32.
    weight: OIHW, or HWIO (KH, KW, C_in, C_out) with layout=WLAYOUT_HWIO (coalesced reads)."""
    lib = _lib.load()
    for t, n in ((x, "x"), (weight, "weight"), (bn_scale, "bn_scale"), (bn_bias, "bn_bias")):
        _require_cuda(t, n)
    _require_numel(x, s.B * s.C_in * s.H * s.W, torch.float32, "x")
    _require_numel(weight, s.C_out * s.C_in * s.KH * s.KW, torch.float32, "weight")
    _require_numel(bn_scale, s.C_out, torch.float32, "bn_scale")
    _require_numel(bn_bias, s.C_out, torch.float32, "bn_bias")
    OH = (s.H + 2 * s.padding - s.KH) // s.stride + 1
    OW = (s.W + 2 * s.padding - s.KW) // s.stride + 1
    if out is None:
        out = torch.empty(s.B, OH, OW, s.C_out, dtype=torch.float32, device=x.device)
    else:
        _require_cuda(out, "out")
        _require_numel(out, s.B * OH * OW * s.C_out, torch.float32, "out")
    d = make_desc(s)
    check(lib.sengine_amd_stem_conv_bn(ctypes.byref(d), _ptr(x), _ptr(weight), int(layout), _ptr(bn_scale),
                                       _ptr(bn_bias), _ptr(out), _stream(x.device)), "stem_conv_bn")
    return out


def stem_conv_bn_lif_pool(s: ConvSpec, x: torch.Tensor, weight_hwio: torch.Tensor, bn_scale: torch.Tensor,
                          bn_bias: torch.Tensor, pool_k: int = 3, pool_stride: int = 2, pool_pad: int = 1,
                          pooled: Optional[torch.Tensor] = None, spikes: Optional[torch.Tensor] = None):
    """Stem conv + folded BN, the neuron of `s` over the output repeated s.T times, and
    MaxPool2d(pool_k, pool_stride, pool_pad) of the spikes, in one launch.  Returns
    (pooled, spikes): int32 spike-bit tensors (s.T*s.B, POH, POW, C_out/32) and, if a
    `spikes` buffer is given, the stem spikes (s.T*s.B, OH, OW, C_out/32) (else None)."""
    lib = _lib.load()
    for t, n in ((x, "x"), (weight_hwio, "weight_hwio"), (bn_scale, "bn_scale"), (bn_bias, "bn_bias")):
        _require_cuda(t, n)
    _require_numel(x, s.B * s.C_in * s.H * s.W, torch.float32, "x")
    _require_numel(weight_hwio, s.C_out * s.C_in * s.KH * s.KW, torch.float32, "weight_hwio")
    _require_numel(bn_scale, s.C_out, torch.float32, "bn_scale")
    _require_numel(bn_bias, s.C_out, torch.float32, "bn_bias")
    OH = (s.H + 2 * s.padding - s.KH) // s.stride + 1
    OW = (s.W + 2 * s.padding - s.KW) // s.stride + 1
    POH = (OH + 2 * pool_pad - pool_k) // pool_stride + 1
    POW = (OW + 2 * pool_pad - pool_k) // pool_stride + 1
    if pooled is None:
        pooled = torch.empty(s.T * s.B, POH, POW, s.C_out // 32, dtype=torch.int32, device=x.device)
    else:
        _require_cuda(pooled, "pooled")
        _require_numel(pooled, s.T * s.B * POH * POW * s.C_out // 32, torch.int32, "pooled")
    if spikes is not None:
        _require_cuda(spikes, "spikes")
        _require_numel(spikes, s.T * s.B * OH * OW * s.C_out // 32, torch.int32, "spikes")
    d = make_desc(s)
    check(lib.sengine_amd_stem_conv_bn_lif_pool(ctypes.byref(d), _ptr(x), _ptr(weight_hwio), _ptr(bn_scale),
                                                _ptr(bn_bias), int(pool_k), int(pool_stride), int(pool_pad),
                                                _ptr(spikes) if spikes is not None else None, _ptr(pooled),
                                                _stream(x.device)), "stem_conv_bn_lif_pool")
    return pooled, spikes


def stem_conv_bn_neuron(s: ConvSpec, x: torch.Tensor, weight_hwio: torch.Tensor, bn_scale: torch.Tensor,
                        bn_bias: torch.Tensor, out: Optional[torch.Tensor] = None, spikes: Optional[torch.Tensor] = None,
                        want_out: bool = True):
    """Stem conv + folded BN (NHWC fp32 `out`, skipped when want_out is False and no `out`
    is given) and the neuron of `s` over that output repeated s.T times (spike bits int32
    (s.T*s.B, OH, OW, C_out/32), the layout of multistep_neuron_repeat on `out`), in one
    launch.  Returns (out or None, spikes)."""
    lib = _lib.load()
    for t, n in ((x, "x"), (weight_hwio, "weight_hwio"), (bn_scale, "bn_scale"), (bn_bias, "bn_bias")):
        _require_cuda(t, n)
    _require_numel(x, s.B * s.C_in * s.H * s.W, torch.float32, "x")
    _require_numel(weight_hwio, s.C_out * s.C_in * s.KH * s.KW, torch.float32, "weight_hwio")
    _require_numel(bn_scale, s.C_out, torch.float32, "bn_scale")
    _require_numel(bn_bias, s.C_out, torch.float32, "bn_bias")
    OH = (s.H + 2 * s.padding - s.KH) // s.stride + 1
    OW = (s.W + 2 * s.padding - s.KW) // s.stride + 1
    if out is None and want_out:
        out = torch.empty(s.B, OH, OW, s.C_out, dtype=torch.float32, device=x.device)
    elif out is not None:
        _require_cuda(out, "out")
        _require_numel(out, s.B * OH * OW * s.C_out, torch.float32, "out")
    if spikes is None:
        spikes = torch.empty(s.T * s.B, OH, OW, s.C_out // 32, dtype=torch.int32, device=x.device)
    else:
        _require_cuda(spikes, "spikes")
        _require_numel(spikes, s.T * s.B * OH * OW * s.C_out // 32, torch.int32, "spikes")
    d = make_desc(s)
    check(lib.sengine_amd_stem_conv_bn_neuron(ctypes.byref(d), _ptr(x), _ptr(weight_hwio), _ptr(bn_scale),
                                              _ptr(bn_bias), _ptr(out) if out is not None else None, _ptr(spikes),
                                              _stream(x.device)), "stem_conv_bn_neuron")
    return out, spikes


def multistep_neuron_repeat(x: torch.Tensor, T: int, neuron: str = "lif", tau: float = 2.0, v_threshold: float = 1.0,
                            v_reset: Optional[float] = 0.0, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Neuron over T steps of the same input x (fp32, n % 32 == 0): spike bits int32 (T, n/32)."""
    lib = _lib.load()
    _require_cuda(x, "x")
    if x.dtype != torch.float32:
        raise SEngineError("multistep_neuron_repeat: x must be fp32")
    n = x.numel()
    if out is None:
        out = torch.empty(T, n // 32, dtype=torch.int32, device=x.device)
    else:
        _require_cuda(out, "out")
        _require_numel(out, T * n // 32, torch.int32, "out")
    hard = v_reset is not None
    check(lib.sengine_amd_multistep_neuron_repeat(int(T), int(n), neuron_code(neuron),
                                                  int(hard), float(tau), float(v_threshold),
                                                  float(v_reset if hard else 0.0), _ptr(x), _ptr(out),
                                                  _stream(x.device)), "multistep_neuron_repeat")
    return out


def maxpool_spikes(x: torch.Tensor, NT: int, H: int, W: int, C: int, k: int = 3, stride: int = 2, pad: int = 1,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Max-pool spike bits (NT, H, W, C/32 words) -> (NT, OH, OW, C/32)."""
    lib = _lib.load()
    _require_cuda(x, "x")
    _require_numel(x, NT * H * W * C // 32, torch.int32, "x")
    OH, OW = (H + 2 * pad - k) // stride + 1, (W + 2 * pad - k) // stride + 1
    if out is None:
        out = torch.empty(NT, OH, OW, C // 32, dtype=torch.int32, device=x.device)
    else:
        _require_cuda(out, "out")
        _require_numel(out, NT * OH * OW * C // 32, torch.int32, "out")
    check(lib.sengine_amd_maxpool_spikes(NT, H, W, C, k, stride, pad, _ptr(x), _ptr(out), _stream(x.device)),
          "maxpool_spikes")
    return out


HEAD_WS_SPLIT = 64  # summing workgroups per image of sengine_amd_sew_head_ws (workspace B * 64 * C)


def sew_head(x: torch.Tensor, T: int, B: int, HW: int, C: int, planes: int, fc_weight: torch.Tensor,
             fc_bias: torch.Tensor, out: Optional[torch.Tensor] = None,
             workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Average pool + mean over T + Linear on `planes`-plane integer activations (planes = 0:
    integer-valued fp16 (T*B, HW, C)) -> (B, N_out) fp32.  fc_weight: (N_out, C) contiguous,
    nn.Linear layout.  With `workspace` (int32, at least B * 64 * C elements) an fp16 stream's
    sums are split over many workgroups per image (sengine_amd_sew_head_ws)."""
    lib = _lib.load()
    for t, n in ((x, "x"), (fc_weight, "fc_weight"), (fc_bias, "fc_bias")):
        _require_cuda(t, n)
    if planes == 0:
        _require_numel(x, T * B * HW * C, torch.float16, "x")
    else:
        _require_numel(x, T * B * HW * planes * C // 32, torch.int32, "x")
    N_out = fc_weight.shape[0]
    _require_numel(fc_weight, N_out * C, torch.float32, "fc_weight")
    _require_numel(fc_bias, N_out, torch.float32, "fc_bias")
    if out is None:
        out = torch.empty(B, N_out, dtype=torch.float32, device=x.device)
    else:
        _require_cuda(out, "out")
        _require_numel(out, B * N_out, torch.float32, "out")
    if workspace is not None:
        _require_cuda(workspace, "workspace")
        if workspace.dtype != torch.int32 or workspace.numel() < B * HEAD_WS_SPLIT * C:
            raise SEngineError(f"workspace: need >= {B * HEAD_WS_SPLIT * C} int32 elements")
        check(lib.sengine_amd_sew_head_ws(T, B, HW, C, planes, _ptr(x), _ptr(fc_weight), _ptr(fc_bias), N_out,
                                          _ptr(out), _ptr(workspace), workspace.numel(), _stream(x.device)),
              "sew_head_ws")
        return out
    check(lib.sengine_amd_sew_head(T, B, HW, C, planes, _ptr(x), _ptr(fc_weight), _ptr(fc_bias), N_out, _ptr(out),
                                   _stream(x.device)), "sew_head")
    return out


def dense_conv_bn(s: ConvSpec, data: torch.Tensor, values: torch.Tensor, bn_scale: torch.Tensor,
                  bn_bias: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Dense Conv + folded BN -> fp32 (T*B, OH, OW, C_out)."""
    lib = _lib.load()
    OH, OW, M, _ = geometry(s)
    d = make_desc(s)
    vb = ctypes.c_size_t()
    check(lib.sengine_amd_dense_blob_bytes(ctypes.byref(d), ctypes.byref(vb)), "dense_blob_bytes")
    for t, n in ((data, "data"), (values, "values"), (bn_scale, "bn_scale"), (bn_bias, "bn_bias")):
        _require_cuda(t, n)
    dt, n_in = _enc_numel(s.in_enc, s.T * s.B * s.H * s.W * s.C_in)
    _require_numel(data, n_in, dt, "data")
    if values.numel() * values.element_size() != vb.value:
        raise SEngineError("dense_conv_bn: weight blob does not match the descriptor")
    _require_numel(bn_scale, s.C_out, torch.float32, "bn_scale")
    _require_numel(bn_bias, s.C_out, torch.float32, "bn_bias")
    if out is None:
        out = torch.empty(s.T * s.B, OH, OW, s.C_out, dtype=torch.float32, device=data.device)
    else:
        _require_cuda(out, "out")
        _require_numel(out, s.T * M * s.C_out, torch.float32, "out")
    check(lib.sengine_amd_dense_conv_bn(ctypes.byref(d), _ptr(data), _ptr(values), _ptr(bn_scale), _ptr(bn_bias),
                                        _ptr(out), _stream(data.device)), "dense_conv_bn")
    return out


def multistep_neuron(x: torch.Tensor, T: int, neuron: str = "lif", tau: float = 2.0, v_threshold: float = 1.0,
                     v_reset: Optional[float] = 0.0, state: Optional[torch.Tensor] = None, out_enc: int = ENC_BITS,
                     h_trace: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Standalone multi-step LIF/IF over T on x (T, ...) fp32 (n = x.numel()/T per step).
    v_reset=None selects soft reset (models/neurons.py:135-137).  Returns spikes as bits
    int32 (T, n/32) or fp16 (T, n)."""
    lib = _lib.load()
    _require_cuda(x, "x")
    if x.dtype != torch.float32 or x.numel() % T:
        raise SEngineError("multistep_neuron: x must be fp32 with T * n elements")
    n = x.numel() // T
    if state is not None:
        _require_cuda(state, "state")
        _require_numel(state, n, torch.float32, "state")
    if h_trace is not None:
        _require_cuda(h_trace, "h_trace")
        _require_numel(h_trace, T * n, torch.float32, "h_trace")
    odt, n_out = _enc_numel(out_enc, T * n)
    if out is None:
        out = torch.empty(n_out, dtype=odt, device=x.device)
    else:
        _require_cuda(out, "out")
        _require_numel(out, n_out, odt, "out")
    hard = v_reset is not None
    check(lib.sengine_amd_multistep_neuron(T, n, neuron_code(neuron), int(hard), float(tau),
                                           float(v_threshold), float(v_reset if hard else 0.0), _ptr(x), _ptr(state),
                                           out_enc, _ptr(out), _ptr(h_trace), _stream(x.device)), "multistep_neuron")
    return out
