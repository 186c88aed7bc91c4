"""Per-node shared objects with the reference's native kernel ABI.

The reference exports every compiled kernel as a standalone .so with `int init(void)` and
`int call(<device pointers in prim_func order>, cudaStream_t)` (sengine/build/export_standalone.py:1-8,37-103),
dlopen'd and called by its C++ executor (sengine/csrc/cpp_executor.cu:631-662,891-916).
export_kernel_so() writes the same two symbols for a kernel object of this build as a
small C shim (compiled with gcc) that bakes the node's descriptor and forwards to
libsengine_amd.so.  The fused node's call() takes the reference's six pointers
(data, weight, state, bn_scale, bn_bias, spikes) + stream, `weight` being the runtime's fp16
(KH, KW, C_in, C_out) tensor (cuda_graph_runtime.py:233-235): the library builds the 2:4
blob on the first call outside capture and reuses it (sengine_amd_fused_call_raw_weight),
so captured calls allocate and synchronise nothing.  call_blob() takes a pre-built
SparseWeight blob (values followed by metadata) instead; `state` may be NULL in both.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import tempfile

from . import _lib, ops
from .build import LIB_DIR, REPO_DIR
from .compiler import DenseConvBNKernel, FusedSparseConvBNLIFKernel

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

_SHIM = r"""
#include <stddef.h>
#include "sengine_amd.h"

static const sengine_conv_lif_desc kDesc = {
  %(T)d, %(B)d, %(C_in)d, %(H)d, %(W)d, %(C_out)d, %(KH)d, %(KW)d, %(S)d, %(S)d, %(P)d, %(P)d, %(D)d, %(D)d,
  %(neuron)d, %(hard)d, %(tau)r, %(vth)r, %(vreset)r, %(in_enc)d, %(out_enc)d, %(planes)d };
static const size_t kValueBytes = %(value_bytes)d;

int init(void) { return sengine_amd_version() > 0 ? 0 : -1; }
%(call)s
"""

_CALL_FUSED = r"""
int call(void* data, void* weight, void* state, void* bn_scale, void* bn_bias, void* spikes, hipStream_t stream) {
  return sengine_amd_fused_call_raw_weight(&kDesc, data, weight, SENGINE_ENC_F16, SENGINE_WLAYOUT_HWIO,
                                           (float*)state, (const float*)bn_scale, (const float*)bn_bias, spikes,
                                           stream);
}
int call_blob(void* data, void* weight, void* state, void* bn_scale, void* bn_bias, void* spikes, hipStream_t stream) {
  return sengine_amd_fused_sparse_conv_bn_lif(&kDesc, data, weight, (const char*)weight + kValueBytes,
                                              (float*)state, (const float*)bn_scale, (const float*)bn_bias,
                                              spikes, NULL, NULL, stream);
}
"""

_CALL_DENSE = r"""
int call(void* data, void* weight, void* bn_scale, void* bn_bias, void* output, hipStream_t stream) {
  return sengine_amd_dense_conv_bn(&kDesc, data, weight, (const float*)bn_scale, (const float*)bn_bias,
                                   (float*)output, stream);
}
"""


def export_kernel_so(kern, output_path: str, in_enc: int = ops.ENC_F16, out_enc: int = ops.ENC_F16,
                     cc: str = "gcc") -> str:
    """Write `output_path` exporting init()/call() for a kernel object from compile_all()."""
    fused = isinstance(kern, FusedSparseConvBNLIFKernel)
    if not fused and not isinstance(kern, DenseConvBNKernel):
        raise TypeError(f"cannot export {type(kern).__name__}")
    s = kern.spec
    d = ops.make_desc(s)
    vb = ctypes.c_size_t()
    mb = ctypes.c_size_t()
    lib = _lib.load()
    if fused:
        _lib.check(lib.sengine_amd_sparse_blob_bytes(ctypes.byref(d), ctypes.byref(vb), ctypes.byref(mb)), "blob bytes")
    src = _SHIM % dict(T=s.T, B=s.B, C_in=s.C_in, H=s.H, W=s.W, C_out=s.C_out, KH=s.KH, KW=s.KW, S=s.stride,
                       P=s.padding, D=s.dilation, neuron=d.neuron, hard=d.hard_reset, in_enc=in_enc,
                       out_enc=out_enc, planes=s.weight_planes, value_bytes=vb.value, call=_CALL_FUSED if fused else _CALL_DENSE,
                       tau=float(s.tau), vth=float(s.v_threshold), vreset=float(s.v_reset))
    os.makedirs(os.path.dirname(os.path.abspath(output_path)), exist_ok=True)
    with tempfile.NamedTemporaryFile("w", suffix=".c", delete=False) as f:
        f.write(src)
        c_path = f.name
    lib_dir = os.path.dirname(_lib.lib_path()) or LIB_DIR
    cmd = [cc, "-O2", "-shared", "-fPIC", "-D__HIP_PLATFORM_AMD__", f"-I{os.path.join(REPO_DIR, 'include')}",
           f"-I{ROCM}/include", c_path, "-o", output_path, f"-L{lib_dir}", "-lsengine_amd", f"-Wl,-rpath,{lib_dir}"]
    try:
        res = subprocess.run(cmd, capture_output=True, text=True)
    finally:
        os.unlink(c_path)
    if res.returncode != 0:
        raise RuntimeError(f"shim compilation failed: {res.stderr[-3000:]}")
    return output_path


def get_call_signature(kern) -> list:
    """(c_type, name) pairs of call(), as export_standalone.get_call_signature (:213-227)."""
    if isinstance(kern, FusedSparseConvBNLIFKernel):
        return [("half_t*", "data"), ("half_t*", "weight"), ("float*", "state"), ("float*", "bn_scale"),
                ("float*", "bn_bias"), ("half_t*", "spikes")]
    return [("half_t*", "data"), ("int16_t*", "weight"), ("float*", "bn_scale"), ("float*", "bn_bias"),
            ("float*", "output")]


def export_all_kernels(kernels: dict, ir, build_dir: str) -> dict:
    """{nid: kernel} -> {nid: .so path}; one .so per distinct kernel object (export_standalone.py:106-210)."""
    os.makedirs(build_dir, exist_ok=True)
    by_obj, out = {}, {}
    for nid, kern in kernels.items():
        if not isinstance(kern, (FusedSparseConvBNLIFKernel, DenseConvBNKernel)):
            continue
        path = by_obj.get(id(kern))
        if path is None:
            path = export_kernel_so(kern, os.path.join(build_dir, f"kern_{nid}.so"))
            by_obj[id(kern)] = path
        out[nid] = path
    return out
