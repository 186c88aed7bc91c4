"""Host-side logic on the CPU: graph passes, weight preparation, the C ABI's exports and
its host-side argument checks (no kernel is launched here)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest
import torch

from oracle import reference_path as ref
from sparsesnn_amd import _lib, ops, passes, sparsity
from sparsesnn_amd.ir import EngineIR, KernelVariant, OpType

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "sengine_amd.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(sengine_amd_\w+)\s*\(", text)))


# ------------------------------------------------------------------------ C ABI

def test_library_exports_every_declared_symbol():
    path = _lib.lib_path()
    assert os.path.exists(path), "build the library first (python -m sparsesnn_amd.build)"
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\b(sengine_amd_\w+)$", out, re.M))
    declared = declared_symbols()
    assert declared, "no declarations parsed from the header"
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    assert set(declared) == set(_lib.SIGNATURES), "ctypes signature table out of sync with the header"


def test_library_loads_and_reports_version():
    lib = _lib.load()
    assert lib.sengine_amd_version() >= 100


def test_desc_struct_layout_matches_header():
    # 19 int32 + 3 float fields, no padding
    assert ctypes.sizeof(_lib.ConvLifDesc) == 22 * 4


def _spec(**kw):
    base = dict(T=4, B=32, C_in=64, H=56, W=56, C_out=64)
    base.update(kw)
    return ops.ConvSpec(**base)


def test_geometry_and_blob_sizes():
    lib = _lib.load()
    assert ops.geometry(_spec()) == (56, 56, 32 * 56 * 56, 576)
    assert ops.geometry(_spec(stride=2)) == (28, 28, 32 * 28 * 28, 576)
    assert ops.geometry(_spec(KH=1, KW=1, padding=0, stride=2)) == (28, 28, 32 * 28 * 28, 64)
    d = ops.make_desc(_spec(C_out=128))
    vb, mb = ctypes.c_size_t(), ctypes.c_size_t()
    assert lib.sengine_amd_sparse_blob_bytes(ctypes.byref(d), ctypes.byref(vb), ctypes.byref(mb)) == 0
    # half the 128 x 576 weights as fp16 values, 2 bits of position per kept value (stored in u32 words)
    assert vb.value == 128 * 576 // 2 * 2 and mb.value == 128 * 576 // 2 * 2 // 16 * 4
    assert lib.sengine_amd_num_groups(ctypes.byref(d)) == 128 * 9 * 16


@pytest.mark.parametrize("field,value,code", [("C_in", 96, -2), ("C_out", 96, -2), ("KH", 0, -2),
                                              ("weight_planes", 3, -2), ("neuron", 7, -2), ("tau", 0.0, -2),
                                              ("T", 3, -3)])
def test_fused_entry_rejects_bad_descriptors_on_host(field, value, code):
    lib = _lib.load()
    d = ops.make_desc(_spec())
    setattr(d, field, value)
    dummy = ctypes.c_void_p(16)  # never dereferenced: validation fails before any launch
    rc = lib.sengine_amd_fused_sparse_conv_bn_lif(ctypes.byref(d), dummy, dummy, dummy, None, dummy, dummy, dummy,
                                                  None, None, None)
    assert rc == code, (rc, lib.sengine_amd_last_error())
    assert lib.sengine_amd_last_error()


def test_null_pointers_rejected_on_host():
    lib = _lib.load()
    d = ops.make_desc(_spec())
    rc = lib.sengine_amd_fused_sparse_conv_bn_lif(ctypes.byref(d), None, None, None, None, None, None, None, None,
                                                  None, None)
    assert rc == -1
    assert lib.sengine_amd_pack_spikes(None, 1, 10, 64, None, None) == -1
    assert lib.sengine_amd_pack_spikes(ctypes.c_void_p(16), 1, 10, 48, ctypes.c_void_p(16), None) == -2
    assert lib.sengine_amd_multistep_neuron(4, 64, 0, 1, 0.0, 1.0, 0.0, ctypes.c_void_p(16), None, 0,
                                            ctypes.c_void_p(16), None, None) == -2


def test_ops_validate_tensors_before_launch():
    spec = _spec(B=1, H=4, W=4)
    with pytest.raises(ops.SEngineError):
        ops.fused_sparse_conv_bn_lif(spec, torch.zeros(4), torch.zeros(4), torch.zeros(4), torch.zeros(4),
                                     torch.zeros(4))  # CPU tensors are refused


def test_export_shim_builds_and_exports_init_call(tmp_path):
    from sparsesnn_amd import compiler, export
    k = compiler.FusedSparseConvBNLIFKernel(_spec(B=1, H=8, W=8), "k")
    so = export.export_kernel_so(k, str(tmp_path / "kern.so"))
    syms = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True).stdout
    assert re.search(r"\bT init$", syms, re.M) and re.search(r"\bT call$", syms, re.M)
    assert [n for _, n in export.get_call_signature(k)] == ["data", "weight", "state", "bn_scale", "bn_bias", "spikes"]


# ------------------------------------------------------------------------ weight preparation

def test_product_prune_matches_oracle_without_ties():
    g = torch.Generator().manual_seed(11)
    w = torch.randn((64, 128, 3, 3), generator=g)
    assert torch.equal(sparsity.prune_conv_2_4(w), ref.prune_conv_2_4(w))
    assert sparsity.validate_2_4_pattern(sparsity.prune_conv_2_4(w))
    assert sparsity.verify_2_4(sparsity.conv_weight_2d(sparsity.prune_conv_2_4(w)))
    w2 = torch.randn((5, 10), generator=g)
    assert torch.equal(sparsity.prune_n_m(w2), ref.prune_n_m(w2))


def test_product_fold_matches_oracle():
    g = torch.Generator().manual_seed(12)
    vec = [torch.rand(64, generator=g) + 0.5 for _ in range(4)]
    s1, b1 = sparsity.fold_batchnorm(*vec, 1e-5)
    s2, b2 = ref.fold_batchnorm(*vec, 1e-5)
    assert np.array_equal(s1.numpy(), s2) and np.array_equal(b1.numpy(), b2)


# ------------------------------------------------------------------------ graph passes

def build_block(T=4, B=2, sparse=True, neuron="lif", cin=64, cout=64, k=3):
    torch.manual_seed(0)
    conv = torch.nn.Conv2d(cin, cout, k, padding=k // 2, bias=False)
    if sparse:
        with torch.no_grad():
            conv.weight.copy_(sparsity.prune_conv_2_4(conv.weight))
    bn = torch.nn.BatchNorm2d(cout).eval()
    ir = EngineIR()
    ir.T = T
    out = passes.add_conv_bn_neuron(ir, "l1", "input", (T * B, cin, 8, 8), conv, bn, neuron)
    return ir, out, conv, bn


def test_passes_route_sparse_conv_to_fused_variant():
    ir, out, conv, bn = build_block()
    stats = passes.optimize_ir(ir)
    assert stats == dict(fused=1, dense=0, unsupported=0, folded=1, groups=1, sparse=1, stems=0, adds=0, heads=0,
                         pools=0, shortcuts=0, real_convs=0, linears=0, padded=0, merged=0, attention=0)
    convs = [n for n in ir.nodes.values() if n.op_type == OpType.Conv2d]
    lifs = [n for n in ir.nodes.values() if n.op_type == OpType.LIF]
    assert not [n for n in ir.nodes.values() if n.op_type == OpType.BatchNorm]
    c, l = convs[0], lifs[0]
    assert c.assigned_kernel == KernelVariant.FusedSparseConvBNLIF
    assert l.assigned_kernel == KernelVariant.ZeroCost
    assert c.extra_attrs["fusion_slice"] == "Conv2d+LIF" and c.extra_attrs["absorbed_nids"] == [l.id]
    s, b = ref.fold_batchnorm(bn.weight.detach(), bn.bias.detach(), bn.running_mean, bn.running_var, bn.eps)
    assert np.array_equal(np.array(c.bn_scale, np.float32), s) and np.array_equal(np.array(c.bn_bias, np.float32), b)
    assert ir.predecessors(l.id) == [c.id]  # BN removed and rewired


def test_passes_route_dense_conv_to_fallback():
    ir, *_ = build_block(sparse=False, neuron="if")
    stats = passes.optimize_ir(ir)
    assert stats["dense"] == 1 and stats["fused"] == 0
    c = [n for n in ir.nodes.values() if n.op_type == OpType.Conv2d][0]
    n = [n for n in ir.nodes.values() if n.op_type == OpType.IF][0]
    assert c.assigned_kernel == KernelVariant.TileLangConvBN and n.assigned_kernel == KernelVariant.CUDAVec4IF


def test_unsupported_shapes_are_not_fused():
    ir, *_ = build_block(cin=48)  # 2:4 but C_in % 64 != 0 and % 32 != 0
    stats = passes.optimize_ir(ir)
    assert stats["unsupported"] == 1


def test_compile_all_caches_kernels_by_shape():
    from sparsesnn_amd.compiler import FusedSparseConvBNLIFKernel, SparseKernelCompiler
    ir, *_ = build_block(B=2)
    passes.optimize_ir(ir)
    kernels = SparseKernelCompiler(ir, batch_size=2).compile_all()
    (nid, kern), = kernels.items()
    assert isinstance(kern, FusedSparseConvBNLIFKernel)
    assert kern.spec.neuron == "lif" and kern.spec.tau == 2.0 and kern.spec.T == 4 and kern.spec.B == 2
    with pytest.raises(ops.SEngineError):
        SparseKernelCompiler(ir, batch_size=3).compile_all()  # T*B mismatch with the graph
