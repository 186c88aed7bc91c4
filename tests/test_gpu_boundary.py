"""GPU: the three drop-in contracts of the fused node.

1. graph-node contract: torch modules -> EngineIR -> optimize_ir -> FusedSparseConvBNLIF;
2. kernel-object contract: compile_all()[nid](data, weight, state, bn_scale, bn_bias),
   called the way sengine/cuda_graph_runtime.py:616-643 calls it (fp16 NHWC in/out,
   HWIO weight tensor as the runtime allocates it, membrane (B*OH*OW, C_out));
3. native ABI: the exported per-node .so, dlopen'd, init() then call(6 ptrs, stream) with
   the runtime's fp16 HWIO weight (call_blob() with a pre-built blob), also captured into a
   hipGraph and replayed with eager work in between.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import reference_path as ref
from sparsesnn_amd import export, ops, passes, sparsity
from sparsesnn_amd.compiler import SparseKernelCompiler
from sparsesnn_amd.ir import EngineIR, KernelVariant
from tests.parity import compare, nhwc_seq

pytestmark = pytest.mark.gpu
T, B, C, H, W, F = 4, 2, 64, 12, 10, 128


def build(neuron="lif"):
    torch.manual_seed(1)
    conv = torch.nn.Conv2d(C, F, 3, padding=1, bias=False)
    with torch.no_grad():
        conv.weight.copy_(sparsity.prune_conv_2_4(conv.weight * 0.5).half().float())
    bn = torch.nn.BatchNorm2d(F).eval()
    with torch.no_grad():
        bn.weight.uniform_(0.5, 1.5)
        bn.bias.normal_(0, 0.1)
        bn.running_mean.normal_(0, 0.1)
        bn.running_var.uniform_(0.5, 1.5)
    ir = EngineIR()
    ir.T = T
    passes.add_conv_bn_neuron(ir, "blk", "x", (T * B, C, H, W), conv, bn, neuron)
    passes.optimize_ir(ir)
    (cid,) = [n.id for n in ir.nodes.values() if n.assigned_kernel == KernelVariant.FusedSparseConvBNLIF]
    return ir, cid, conv, bn


def inputs(dev, seed=3):
    g = torch.Generator().manual_seed(seed)
    x = torch.bernoulli(torch.full((T, B, C, H, W), 0.25), generator=g)
    return x, x.permute(0, 1, 3, 4, 2).reshape(T * B, H, W, C).contiguous().half().to(dev)


def oracle(x, conv, bn, neuron="lif"):
    b = ref.BNParams(bn.weight.detach(), bn.bias.detach(), bn.running_mean, bn.running_var, bn.eps)
    return ref.fused_layer(x, conv.weight.detach(), b, 1, 1, 1, neuron, 2.0, 1.0, 0.0)


def check(spikes_nhwc, r):
    rep = compare(nhwc_seq(spikes_nhwc, T), None, r.spikes.numpy(), r.h.numpy(), 1.0)
    assert rep.ok, str(rep)


@pytest.mark.parametrize("neuron", ["lif", "if"])
def test_kernel_object_contract(dev, neuron):
    ir, cid, conv, bn = build(neuron)
    node = ir.nodes[cid]
    kern = SparseKernelCompiler(ir, batch_size=B).compile_all()[cid]
    x, data = inputs(dev)
    w_hwio = torch.from_numpy(ir.weights[node.weight_info.name]).permute(2, 3, 1, 0).contiguous().half().to(dev)
    sc = torch.tensor(node.bn_scale, dtype=torch.float32, device=dev)
    bi = torch.tensor(node.bn_bias, dtype=torch.float32, device=dev)
    mem = torch.zeros(B * H * W, F, device=dev)
    spikes = kern(data, w_hwio, mem, sc, bi)
    assert spikes.dtype == torch.float16 and tuple(spikes.shape) == (T * B, H, W, F)
    r = oracle(x, conv, bn, neuron)
    check(spikes.float().cpu(), r)
    # final membrane written back as (B*OH*OW, C_out)
    v = mem.view(B, H, W, F).permute(0, 3, 1, 2).cpu()
    assert torch.allclose(v, r.v_final, atol=1e-4)
    # four-argument form: no membrane
    spikes4 = kern(data, w_hwio, sc, bi)
    assert torch.equal(spikes4.cpu(), spikes.cpu())


def test_exported_so_call_and_graph_replay(dev, tmp_path):
    """call() takes the runtime's fp16 (KH, KW, C_in, C_out) weight: the first (eager) call
    builds the 2:4 blob, later calls and a captured call reuse it; call_blob() takes a pre-built
    blob; a weight first seen inside a capture is refused with -4."""
    from sparsesnn_amd import _lib
    ir, cid, conv, bn = build()
    node = ir.nodes[cid]
    kern = SparseKernelCompiler(ir, batch_size=B).compile_all()[cid]
    so_path = export.export_all_kernels({cid: kern}, ir, str(tmp_path))[cid]
    so = ctypes.CDLL(so_path)
    so.init.restype = ctypes.c_int
    for fn in (so.call, so.call_blob):
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_void_p] * 7
    assert so.init() == 0
    w_oihw = torch.from_numpy(ir.weights[node.weight_info.name])
    w_hwio = w_oihw.permute(2, 3, 1, 0).contiguous().half().to(dev)
    sw = kern.prepare_weight(w_oihw.to(dev))
    sc = torch.tensor(node.bn_scale, dtype=torch.float32, device=dev)
    bi = torch.tensor(node.bn_bias, dtype=torch.float32, device=dev)
    x, data = inputs(dev, seed=4)
    mem = torch.zeros(B * H * W, F, device=dev)
    out = torch.empty(T * B, H, W, F, dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream(dev)
    try:
        def call(fn=so.call, w=w_hwio, s=stream):
            return fn(data.data_ptr(), w.data_ptr(), mem.data_ptr(), sc.data_ptr(), bi.data_ptr(), out.data_ptr(),
                      s.cuda_stream)

        assert call() == 0
        torch.cuda.synchronize()
        r = oracle(x, conv, bn)
        check(out.float().cpu(), r)
        eager = out.clone()
        assert torch.allclose(mem.view(B, H, W, F).permute(0, 3, 1, 2).cpu(), r.v_final, atol=1e-4)
        # the pre-built blob gives the same spikes
        mem.zero_()
        out.fill_(7.0)
        assert call(so.call_blob, sw) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, eager)

        # capture call() into a hipGraph; membranes are zeroed by a fill kernel before each replay
        g = torch.cuda.CUDAGraph()
        mem.zero_()
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            rc = call(s=torch.cuda.current_stream(dev))
        assert rc == 0
        for i in range(4):
            out.fill_(7.0)
            mem.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {i} differs"
            _ = (torch.ones(1000, device=dev) * i).sum().item()  # eager work between replays

        # a weight never called eagerly cannot be prepared inside a capture
        w_new = w_hwio.clone()
        g2 = torch.cuda.CUDAGraph()
        torch.cuda.synchronize()
        with torch.cuda.graph(g2):
            out.fill_(0.0)
            rc = call(w=w_new, s=torch.cuda.current_stream(dev))
        assert rc == -4, rc
        assert "capture" in _lib.load().sengine_amd_last_error().decode()
        # ... and is served once it has been seen eagerly
        mem.zero_()
        assert call(w=w_new) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    finally:
        torch.cuda.synchronize()
        assert _lib.load().sengine_amd_release_weights() == 0


def test_raw_weight_rejects_dense(dev):
    """A weight that is not 2:4 along C_in is refused (-5) and leaves no blob behind."""
    from sparsesnn_amd import _lib
    ir, cid, conv, bn = build()
    node = ir.nodes[cid]
    kern = SparseKernelCompiler(ir, batch_size=B).compile_all()[cid]
    dense = torch.randn(3, 3, C, F, device=dev).half()
    data = torch.zeros(T * B, H, W, C, dtype=torch.float16, device=dev)
    sc = torch.ones(F, device=dev)
    bi = torch.zeros(F, device=dev)
    out = torch.empty(T * B, H, W, F, dtype=torch.float16, device=dev)
    d = ops.make_desc(kern.spec_for(ops.ENC_F16, ops.ENC_F16))
    lib = _lib.load()
    try:
        rc = lib.sengine_amd_fused_call_raw_weight(ctypes.byref(d), data.data_ptr(), dense.data_ptr(), ops.ENC_F16,
                                                   ops.WLAYOUT_HWIO, None, sc.data_ptr(), bi.data_ptr(),
                                                   out.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
        assert rc == -5, rc
        assert "2:4" in lib.sengine_amd_last_error().decode()
        # refused again on the next call: nothing was cached
        rc = lib.sengine_amd_prepare_weight(ctypes.byref(d), dense.data_ptr(), ops.ENC_F16, ops.WLAYOUT_HWIO,
                                            torch.cuda.current_stream(dev).cuda_stream)
        assert rc == -5, rc
    finally:
        torch.cuda.synchronize()
        assert _lib.load().sengine_amd_release_weights() == 0


def test_raw_weight_follows_the_weight_bytes(dev, tmp_path):
    """The raw-weight call() caches a 2:4 blob per weight address, but the reference reads the
    weight on every call: a weight freed and replaced by a different one at the same address
    (the caching allocator hands the block straight back), or updated in place, must give the
    new weight's spikes on the next eager call -- and a graph captured before the update replays
    the refreshed blob once an eager call has seen the new bytes."""
    from sparsesnn_amd import _lib
    ir, cid, conv, bn = build()
    node = ir.nodes[cid]
    kern = SparseKernelCompiler(ir, batch_size=B).compile_all()[cid]
    so = ctypes.CDLL(export.export_all_kernels({cid: kern}, ir, str(tmp_path))[cid])
    so.init.restype = ctypes.c_int
    so.call.restype = ctypes.c_int
    so.call.argtypes = [ctypes.c_void_p] * 7
    assert so.init() == 0
    w_oihw = torch.from_numpy(ir.weights[node.weight_info.name]).float()
    sc = torch.tensor(node.bn_scale, dtype=torch.float32, device=dev)
    bi = torch.tensor(node.bn_bias, dtype=torch.float32, device=dev)
    x, data = inputs(dev, seed=5)
    mem = torch.zeros(B * H * W, F, device=dev)
    out = torch.empty(T * B, H, W, F, dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream(dev)

    def hwio(w):
        return w.permute(2, 3, 1, 0).contiguous().half().to(dev)

    def call(w, s=stream):
        mem.zero_()
        return so.call(data.data_ptr(), w.data_ptr(), mem.data_ptr(), sc.data_ptr(), bi.data_ptr(), out.data_ptr(),
                       s.cuda_stream)

    def expect(w, what):
        c = torch.nn.Conv2d(C, F, 3, padding=1, bias=False)
        with torch.no_grad():
            c.weight.copy_(w)
        r = oracle(x, c, bn)
        rep = compare(nhwc_seq(out.float().cpu(), T), None, r.spikes.numpy(), r.h.numpy(), 1.0)
        assert rep.ok, f"{what}: {rep}"
        assert torch.allclose(mem.view(B, H, W, F).permute(0, 3, 1, 2).cpu(), r.v_final, atol=1e-4), what
        return r

    # three different 2:4 weights with the same shape (same magnitudes, other signs / order)
    w_a = w_oihw
    w_b = -w_oihw
    w_c = torch.roll(w_oihw, shifts=1, dims=0)  # output channels permuted
    try:
        wa = hwio(w_a)
        addr = wa.data_ptr()
        assert call(wa) == 0
        torch.cuda.synchronize()
        r_a = expect(w_a, "first weight")
        del wa  # freed: the caching allocator keeps the block for the next request of this size
        wb = hwio(w_b)
        assert wb.data_ptr() == addr, "the allocator did not reuse the address (the case this test is about)"
        assert call(wb) == 0
        torch.cuda.synchronize()
        r_b = expect(w_b, "different weight at a reused address")
        assert float((r_a.v_final - r_b.v_final).abs().max()) > 0.1  # the two weights are told apart

        # a graph captured over wb; then wb updated in place (same address, same tensor)
        g = torch.cuda.CUDAGraph()
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            rc = so.call(data.data_ptr(), wb.data_ptr(), mem.data_ptr(), sc.data_ptr(), bi.data_ptr(),
                         out.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
        assert rc == 0
        wb.copy_(hwio(w_c))
        assert call(wb) == 0  # eager: sees the new bytes, rebuilds the blob in place
        torch.cuda.synchronize()
        expect(w_c, "weight updated in place")
        for i in range(3):  # the captured graph replays the refreshed blob
            out.fill_(7.0)
            mem.zero_()
            g.replay()
            torch.cuda.synchronize()
            expect(w_c, f"graph replay {i} after the in-place update")
            _ = (torch.ones(1000, device=dev) * i).sum().item()
        # a dense weight written over it is refused on the next eager call, and by captured ones
        wb.copy_(torch.randn(3, 3, C, F, device=dev).half())
        assert call(wb) == -5
        assert "2:4" in _lib.load().sengine_amd_last_error().decode()
    finally:
        torch.cuda.synchronize()
        assert _lib.load().sengine_amd_release_weights() == 0


@pytest.mark.gpu
def test_calibrate_stream_modes(dev):
    """The bandwidth probes move what they claim: the copy and the non-temporal copy reproduce
    the source, and the read-only stream's per-thread checksums fold to the XOR of every source
    word (the rest of the destination untouched); bad modes and misaligned buffers are refused."""
    from sparsesnn_amd import _lib
    lib = _lib.load()
    n = (1 << 20) + 48  # 16-byte pieces that do not fill the last trip of the grid
    src = torch.randint(-2**31, 2**31 - 1, (n,), dtype=torch.int32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    for mode in (0, 1, 2):
        dst = torch.zeros_like(src)
        assert lib.sengine_amd_calibrate_stream(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()),
                                                4 * n, mode, stream) == 0
        torch.cuda.synchronize(dev)
        if mode < 2:
            assert torch.equal(dst, src), mode
        else:
            h = src.cpu().numpy().view(np.uint32)
            assert np.bitwise_xor.reduce(dst.cpu().numpy().view(np.uint32)) == np.bitwise_xor.reduce(h)
    dst = torch.zeros_like(src)
    assert lib.sengine_amd_calibrate_stream(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()),
                                            4 * n, 3, stream) == -2
    assert lib.sengine_amd_calibrate_stream(ctypes.c_void_p(src.data_ptr() + 4), ctypes.c_void_p(dst.data_ptr()),
                                            4 * n - 16, 1, stream) == -2
