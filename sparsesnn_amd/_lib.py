"""ctypes binding of libsengine_amd.so (the C ABI of include/sengine_amd.h).

Loading fails loudly: there is no CPU or PyTorch fallback behind these entry points.
"""
from __future__ import annotations

import ctypes
import os
import threading

from .build import LIB_PATH

ENC_BITS, ENC_F16, ENC_F32 = 0, 1, 2
NEURON_LIF, NEURON_IF, NEURON_MS = 0, 1, 2
WLAYOUT_OIHW, WLAYOUT_HWIO = 0, 1


class ConvLifDesc(ctypes.Structure):
    """Mirror of ``sengine_conv_lif_desc`` (field order and types must match the header)."""

    _fields_ = [
        ("T", ctypes.c_int32), ("B", ctypes.c_int32),
        ("C_in", ctypes.c_int32), ("H", ctypes.c_int32), ("W", ctypes.c_int32), ("C_out", ctypes.c_int32),
        ("KH", ctypes.c_int32), ("KW", ctypes.c_int32),
        ("stride_h", ctypes.c_int32), ("stride_w", ctypes.c_int32),
        ("pad_h", ctypes.c_int32), ("pad_w", ctypes.c_int32),
        ("dil_h", ctypes.c_int32), ("dil_w", ctypes.c_int32),
        ("neuron", ctypes.c_int32), ("hard_reset", ctypes.c_int32),
        ("tau", ctypes.c_float), ("v_threshold", ctypes.c_float), ("v_reset", ctypes.c_float),
        ("in_enc", ctypes.c_int32), ("out_enc", ctypes.c_int32), ("weight_planes", ctypes.c_int32),
    ]


_P = ctypes.c_void_p
_DP = ctypes.POINTER(ConvLifDesc)
_I32, _I64, _F = ctypes.c_int32, ctypes.c_int64, ctypes.c_float
_SZP = ctypes.POINTER(ctypes.c_size_t)

# name -> (restype, argtypes); every symbol declared in include/sengine_amd.h
SIGNATURES = {
    "sengine_amd_version": (ctypes.c_int, []),
    "sengine_amd_last_error": (ctypes.c_char_p, []),
    "sengine_amd_set_fused_kernel": (ctypes.c_int, [_I32]),
    "sengine_amd_conv_geometry": (ctypes.c_int, [_DP, ctypes.POINTER(_I32), ctypes.POINTER(_I32),
                                                 ctypes.POINTER(_I64), ctypes.POINTER(_I64)]),
    "sengine_amd_sparse_blob_bytes": (ctypes.c_int, [_DP, _SZP, _SZP]),
    "sengine_amd_dense_blob_bytes": (ctypes.c_int, [_DP, _SZP]),
    "sengine_amd_compress_2_4": (ctypes.c_int, [_DP, _P, _I32, _I32, _P, _P, _P, _P]),
    "sengine_amd_tail_blob_bytes": (ctypes.c_int, [_DP, _SZP, _SZP]),
    "sengine_amd_compress_2_4_tail": (ctypes.c_int, [_DP, _P, _I32, _I32, _P, _P, _P, _P]),
    "sengine_amd_fused_sparse_conv_bn_lif_tail": (ctypes.c_int, [_DP, _P, _P, _P, _P, _P, _P, _P, _P]),
    "sengine_amd_num_groups": (ctypes.c_int64, [_DP]),
    "sengine_amd_pack_dense_weights": (ctypes.c_int, [_DP, _P, _I32, _I32, _P, _P]),
    "sengine_amd_fused_sparse_conv_bn_lif": (ctypes.c_int, [_DP, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "sengine_amd_fused_plan": (ctypes.c_int, [_DP, _I32, ctypes.c_char_p, ctypes.c_size_t]),
    "sengine_amd_fused_sparse_conv_bn_lif_split": (ctypes.c_int, [_DP, _P, _P, _P, _P, _P, _P, _P, _I32, _P]),
    "sengine_amd_calibrate_smfmac": (ctypes.c_int, [_I32, _I32, _P, _P]),
    "sengine_amd_fused_call_raw_weight": (ctypes.c_int, [_DP, _P, _P, _I32, _I32, _P, _P, _P, _P, _P]),
    "sengine_amd_prepare_weight": (ctypes.c_int, [_DP, _P, _I32, _I32, _P]),
    "sengine_amd_release_weights": (ctypes.c_int, []),
    "sengine_amd_calibrate_copy": (ctypes.c_int, [_P, _P, _I64, _P]),
    "sengine_amd_calibrate_stream": (ctypes.c_int, [_P, _P, _I64, _I32, _P]),
    "sengine_amd_fused_sparse_conv_bn_lif_pair": (ctypes.c_int, [_DP, _DP, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                                                  _P, _P]),
    "sengine_amd_fused_sparse_conv_bn_lif_add": (ctypes.c_int, [_DP, _P, _P, _P, _P, _P, _P, _P, _I32, _P, _I32,
                                                                _P]),
    "sengine_amd_stem_conv_bn": (ctypes.c_int, [_DP, _P, _P, _I32, _P, _P, _P, _P]),
    "sengine_amd_fused_sparse_conv_bn_add_neuron": (ctypes.c_int, [_DP, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "sengine_amd_real_conv_bn": (ctypes.c_int, [_DP, _P, _I32, _P, _I32, _P, _P, _P, _P]),
    "sengine_amd_ssa_kv": (ctypes.c_int, [_I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P]),
    "sengine_amd_ssa_attend_neuron": (ctypes.c_int, [_I32, _I32, _I32, _I32, _I32, _F, _I32, _I32, _F, _F, _F,
                                                     _P, _P, _P, _P]),
    "sengine_amd_ssa_attention_noalloc": (ctypes.c_int, [_I32, _I32, _I32, _I32, _I32, _F, _I32, _I32, _F, _F, _F,
                                                         _P, _P, _P, _P, _P]),
    "sengine_amd_stem_conv_bn_lif_pool": (ctypes.c_int, [_DP, _P, _P, _P, _P, _I32, _I32, _I32, _P, _P, _P]),
    "sengine_amd_stem_conv_bn_neuron": (ctypes.c_int, [_DP, _P, _P, _P, _P, _P, _P, _P]),
    "sengine_amd_multistep_neuron_repeat": (ctypes.c_int, [_I32, _I64, _I32, _I32, _F, _F, _F, _P, _P, _P]),
    "sengine_amd_maxpool_spikes": (ctypes.c_int, [_I32, _I32, _I32, _I32, _I32, _I32, _I32, _P, _P, _P]),
    "sengine_amd_sew_head": (ctypes.c_int, [_I32, _I32, _I32, _I32, _I32, _P, _P, _P, _I32, _P, _P]),
    "sengine_amd_sew_head_ws": (ctypes.c_int, [_I32, _I32, _I32, _I32, _I32, _P, _P, _P, _I32, _P, _P, _I64, _P]),
    "sengine_amd_dense_conv_bn": (ctypes.c_int, [_DP, _P, _P, _P, _P, _P, _P]),
    "sengine_amd_multistep_neuron": (ctypes.c_int, [_I32, _I64, _I32, _I32, _F, _F, _F, _P, _P, _I32, _P, _P, _P]),
    "sengine_amd_pack_spikes": (ctypes.c_int, [_P, _I32, _I64, _I32, _P, _P]),
    "sengine_amd_unpack_spikes": (ctypes.c_int, [_P, _I64, _I32, _P, _I32, _P]),
}

_lib = None
_lock = threading.Lock()


class SEngineError(RuntimeError):
    """Raised when an entry point of libsengine_amd reports an error."""


def lib_path() -> str:
    return os.environ.get("SENGINE_AMD_LIB", LIB_PATH)


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = lib_path()
            if not os.path.exists(path):
                raise SEngineError(
                    f"{path} is missing: build it with `python -m sparsesnn_amd.build` "
                    "(the sengine_amd ops have no fallback implementation)")
            lib = ctypes.CDLL(path)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc == 0:
        return
    lib = load()
    if rc < 0:
        msg = lib.sengine_amd_last_error().decode()
        raise SEngineError(f"{what}: {msg} (code {rc})")
    raise SEngineError(f"{what}: HIP error {rc}")
