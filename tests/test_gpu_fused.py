"""GPU parity of the fused 2:4-sparse Conv+BN+LIF kernel against the CPU oracle.

Every case runs the reference PyTorch path (oracle.reference_path) on the CPU and the
HIP kernel through the C ABI on the same seeded inputs, then applies the acceptance
rule of tests/parity.py.
"""
import dataclasses
import os

import numpy as np
import pytest
import torch

from oracle import packing as pk
from oracle import reference_path as ref
from sparsesnn_amd import ops
from tests.parity import compare, nhwc_seq

pytestmark = pytest.mark.gpu


def run_case(dev, case: ref.LayerCase, neuron="lif", tau=2.0, v_th=1.0, v_reset=0.0, planes=1,
             in_enc=ops.ENC_BITS, out_enc=ops.ENC_BITS, v0=None, layout=ops.WLAYOUT_OIHW, traces=True, tail=False):
    """One fused call against the oracle.  traces=True also records the per-step membrane and
    BN output (which selects the generic epilogue); traces=False runs the call as an engine
    does (the fast epilogue where the neuron allows it) and compares spikes and, with v0, the
    final membrane.  tail: the paired-tail call (the case's last 32 input channels must have
    zero weights).  Returns (report, BN-output error or None, oracle result, final state)."""
    T, B, C_in, H, W = case.x_seq.shape
    C_out, _, KH, KW = case.w.shape
    hard = v_reset is not None
    spec = ops.ConvSpec(T=T, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=KH, KW=KW, stride=case.stride,
                        padding=case.padding, neuron=neuron, hard_reset=hard, tau=tau, v_threshold=v_th,
                        v_reset=v_reset if hard else 0.0, in_enc=in_enc, out_enc=out_enc, weight_planes=planes)
    OH, OW, M, _ = ops.geometry(spec)
    w_dev = case.w.to(dev) if layout == ops.WLAYOUT_OIHW else case.w.permute(2, 3, 1, 0).contiguous().to(dev)
    values, meta, _ = ops.compress_2_4(spec, w_dev, layout, tail=tail)
    scale, bias = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
    scale_d = torch.from_numpy(scale).to(dev)
    bias_d = torch.from_numpy(bias).to(dev)
    x_nhwc = case.x_seq.permute(0, 1, 3, 4, 2).reshape(T * B, H, W, C_in).contiguous()
    if in_enc == ops.ENC_BITS:
        data = torch.from_numpy(pk.seq_to_nhwc_bits(case.x_seq.numpy()).view(np.int32)).to(dev)
    else:
        data = x_nhwc.half().to(dev)
    state = None
    if v0 is not None:
        state = v0.permute(0, 2, 3, 1).reshape(M, C_out).contiguous().to(dev)
    h_tr = torch.empty(T, M, C_out, dtype=torch.float32, device=dev) if traces else None
    x_tr = torch.empty(T, M, C_out, dtype=torch.float32, device=dev) if traces else None
    if tail:
        assert not traces
        out = ops.fused_sparse_conv_bn_lif_tail(spec, data, values, meta, scale_d, bias_d, state=state)
    else:
        out = ops.fused_sparse_conv_bn_lif(spec, data, values, meta, scale_d, bias_d, state=state,
                                           h_trace=h_tr, x_trace=x_tr)
    torch.cuda.synchronize()
    if out_enc == ops.ENC_BITS:
        s_gpu = pk.unpack_bits(out.cpu().numpy().view(np.uint32).reshape(-1, C_out // 32), C_out)
        s_gpu = torch.from_numpy(s_gpu.reshape(T * B, OH, OW, C_out))
    else:
        s_gpu = out.float().cpu()
    r = ref.fused_layer(case.x_seq, case.w, case.bn, case.stride, case.padding, 1, neuron, tau, v_th, v_reset, v0)
    h_gpu = nhwc_seq(h_tr.view(T * B, OH, OW, C_out), T) if traces else None
    rep = compare(nhwc_seq(s_gpu, T), h_gpu, r.spikes.numpy(), r.h.numpy(), v_th)
    x_err = None
    if traces:
        x_gpu = nhwc_seq(x_tr.view(T * B, OH, OW, C_out), T)
        x_err = float(np.max(np.abs(x_gpu - r.x.numpy())))
    v_fin = None
    if state is not None:
        v_fin = state.view(B, OH, OW, C_out).permute(0, 3, 1, 2).cpu()
    return rep, x_err, r, v_fin


def test_cfg0_lif_bits(dev):
    case = ref.make_layer_case(0, T=4, B=1, C_in=64, C_out=64, H=32, W=32, k=3)
    rep, x_err, r, _ = run_case(dev, case, planes=2)
    print(rep, "x_err", x_err, "spike rate", float(r.spikes.mean()))
    assert rep.ok, str(rep)
    assert x_err < 1e-4


@pytest.mark.parametrize("planes", [1, 2])
@pytest.mark.parametrize("in_enc,out_enc", [(ops.ENC_BITS, ops.ENC_BITS), (ops.ENC_F16, ops.ENC_F16),
                                            (ops.ENC_BITS, ops.ENC_F16), (ops.ENC_F16, ops.ENC_BITS)])
def test_encodings(dev, planes, in_enc, out_enc):
    case = ref.make_layer_case(1, T=4, B=2, C_in=64, C_out=128, H=10, W=12, k=3, fp16_weights=(planes == 1))
    rep, x_err, _, _ = run_case(dev, case, planes=planes, in_enc=in_enc, out_enc=out_enc)
    print(rep, x_err)
    assert rep.ok, str(rep)


@pytest.mark.parametrize("k,stride,pad", [(3, 1, 1), (3, 2, 1), (1, 1, 0), (1, 2, 0), (3, 1, 0), (5, 2, 2)])
def test_shapes(dev, k, stride, pad):
    case = ref.make_layer_case(2 + k + stride, T=4, B=3, C_in=128, C_out=64, H=13, W=11, k=k, stride=stride,
                               padding=pad, fp16_weights=True)
    rep, x_err, _, _ = run_case(dev, case)
    print(rep, x_err)
    assert rep.ok, str(rep)


@pytest.mark.parametrize("T", [1, 2, 8])
def test_timesteps(dev, T):
    case = ref.make_layer_case(10 + T, T=T, B=2, C_in=64, C_out=64, H=9, W=9, k=3, fp16_weights=True)
    rep, _, _, _ = run_case(dev, case)
    assert rep.ok, str(rep)


@pytest.mark.parametrize("neuron,tau,v_reset", [("if", 2.0, 0.0), ("lif", 2.0, None), ("if", 2.0, None),
                                                ("lif", 3.0, 0.0), ("lif", 1.5, 0.2), ("lif", 4.0, None)])
def test_neuron_variants(dev, neuron, tau, v_reset):
    case = ref.make_layer_case(20, T=4, B=2, C_in=64, C_out=64, H=8, W=8, k=3, fp16_weights=True, p_spike=0.3)
    rep, _, r, _ = run_case(dev, case, neuron=neuron, tau=tau, v_reset=v_reset, v_th=0.5)
    print(neuron, tau, v_reset, rep, float(r.spikes.mean()))
    assert rep.ok, str(rep)


def test_state_in_out(dev):
    case = ref.make_layer_case(30, T=4, B=2, C_in=64, C_out=64, H=6, W=7, k=3, fp16_weights=True)
    g = torch.Generator().manual_seed(5)
    v0 = torch.rand((2, 64, 6, 7), generator=g) * 0.9
    rep, _, r, v_fin = run_case(dev, case, v0=v0)
    assert rep.ok, str(rep)
    assert torch.allclose(v_fin, r.v_final, rtol=1e-3, atol=1e-3)


def test_hwio_layout(dev):
    case = ref.make_layer_case(31, T=4, B=1, C_in=64, C_out=64, H=8, W=8, k=3, fp16_weights=True)
    rep, _, _, _ = run_case(dev, case, layout=ops.WLAYOUT_HWIO)
    assert rep.ok, str(rep)


@pytest.mark.parametrize("traces", [True, False])
@pytest.mark.parametrize("kernel", ["direct", "lds", "auto", "tile"])
@pytest.mark.parametrize("k,stride,pad,B,C_in,C_out,H,W", [(3, 1, 1, 5, 64, 128, 13, 11), (3, 2, 1, 3, 128, 64, 15, 9),
                                                           (1, 1, 0, 2, 256, 192, 7, 7), (1, 2, 0, 2, 64, 64, 9, 10)])
def test_bit_kernels_agree_and_match_oracle(dev, kernel, k, stride, pad, B, C_in, C_out, H, W, traces):
    """Every spike-bit kernel (halo-tiled via 'auto' where eligible, LDS-staged, direct-gather)
    against the oracle, on shapes whose position count is not a multiple of the workgroup tile."""
    ops.set_fused_kernel(kernel)
    try:
        case = ref.make_layer_case(40 + k + stride + B, T=4, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=k,
                                   stride=stride, padding=pad, fp16_weights=True)
        rep, x_err, _, v_fin = run_case(dev, case, traces=traces)
        assert rep.ok, str(rep)
        assert x_err is None or x_err < 1e-4
    finally:
        ops.set_fused_kernel("auto")


@pytest.mark.parametrize("traces", [True, False])
@pytest.mark.parametrize("tile", ["0", "1", "2"])
@pytest.mark.parametrize("H,W,C_in,C_out,B", [(13, 11, 64, 64, 2), (7, 7, 128, 128, 3), (28, 14, 192, 64, 1),
                                              (4, 17, 64, 192, 2)])
def test_halo_tiles_against_oracle(dev, tile, H, W, C_in, C_out, B, traces):
    """3x3 tile kernel with each tile shape forced (0: 8x8, 1: 14x4, 2: 7x7), on images that
    leave ragged tiles, one to three input-channel chunks and several output-channel groups."""
    import os
    os.environ["SENGINE_AMD_TILE_SHAPE"] = tile
    ops.set_fused_kernel("tile")  # small test shapes would otherwise take the small-M kernel
    try:
        case = ref.make_layer_case(60 + H + W + C_in // 64, T=4, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=3,
                                   fp16_weights=True)
        rep, x_err, _, _ = run_case(dev, case, traces=traces)
        assert rep.ok, str(rep)
        assert x_err is None or x_err < 1e-4
        rep2, _, _, _ = run_case(dev, case, neuron="if", v_th=0.5, v_reset=None, out_enc=ops.ENC_F16, traces=traces)
        assert rep2.ok, str(rep2)
    finally:
        ops.set_fused_kernel("auto")
        del os.environ["SENGINE_AMD_TILE_SHAPE"]


@pytest.mark.parametrize("traces", [True, False])
@pytest.mark.parametrize("T", [1, 2])
@pytest.mark.parametrize("neuron,v_reset", [("lif", 0.0), ("if", 0.0), ("lif", None)])
def test_halo_short_sequences_and_state(dev, T, neuron, v_reset, traces):
    case = ref.make_layer_case(70 + T, T=T, B=2, C_in=128, C_out=64, H=9, W=10, k=3, fp16_weights=True,
                               p_spike=0.3)
    g = torch.Generator().manual_seed(9)
    v0 = torch.rand((2, 64, 9, 10), generator=g) * 0.5
    ops.set_fused_kernel("tile")  # small test shapes would otherwise take the small-M kernel
    try:
        rep, _, r, v_fin = run_case(dev, case, neuron=neuron, v_reset=v_reset, v_th=0.6, v0=v0, traces=traces)
    finally:
        ops.set_fused_kernel("auto")
    assert rep.ok, str(rep)
    assert torch.allclose(v_fin, r.v_final, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("traces", [True, False])
@pytest.mark.parametrize("gpw", ["1", "2"])
@pytest.mark.parametrize("k,stride,H,W,C_in,C_out,B", [(3, 1, 9, 10, 128, 128, 2), (1, 1, 7, 9, 256, 256, 3),
                                                       (1, 2, 11, 10, 128, 128, 2), (1, 1, 5, 5, 64, 192, 1)])
def test_tile_channel_blocking(dev, gpw, k, stride, H, W, C_in, C_out, B, traces):
    """Tile kernels with one or two 64-channel groups per wave (SENGINE_AMD_TILE_GPW), for
    3x3 halo tiles and flat 1x1 tiles (stride 1 and 2), against the oracle."""
    import os
    os.environ["SENGINE_AMD_TILE_GPW"] = gpw
    ops.set_fused_kernel("tile")  # small test shapes would otherwise take the small-M kernel
    try:
        case = ref.make_layer_case(80 + k + stride + C_in // 64, T=4, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=k,
                                   stride=stride, padding=k // 2, fp16_weights=True)
        rep, x_err, _, _ = run_case(dev, case, traces=traces)
        assert rep.ok, str(rep)
        assert x_err is None or x_err < 1e-4
        rep2, _, _, _ = run_case(dev, case, neuron="if", v_th=0.5, v_reset=0.0, traces=traces)
        assert rep2.ok, str(rep2)
    finally:
        ops.set_fused_kernel("auto")
        del os.environ["SENGINE_AMD_TILE_GPW"]


@pytest.mark.parametrize("traces", [True, False])
@pytest.mark.parametrize("ksplit", ["1", "2"])
@pytest.mark.parametrize("shape", ["0", "1", "2"])
@pytest.mark.parametrize("H,W,C_in,C_out,B", [(7, 7, 256, 128, 3), (13, 11, 128, 64, 2), (9, 16, 512, 64, 1)])
def test_tile_reduction_split(dev, ksplit, shape, H, W, C_in, C_out, B, traces):
    """3x3 halo tiles with the reduction split over two wave sets (SENGINE_AMD_TILE_KSPLIT),
    each tile shape, LIF (fast epilogue) and IF with state (generic epilogue), against the oracle."""
    import os
    os.environ["SENGINE_AMD_TILE_KSPLIT"] = ksplit
    os.environ["SENGINE_AMD_TILE_SHAPE"] = shape
    ops.set_fused_kernel("tile")  # small test shapes would otherwise take the small-M kernel
    try:
        case = ref.make_layer_case(110 + H + C_in // 64, T=4, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=3,
                                   fp16_weights=True, p_spike=0.2)
        rep, x_err, _, _ = run_case(dev, case, traces=traces)
        assert rep.ok, str(rep)
        assert x_err is None or x_err < 1e-4
        g = torch.Generator().manual_seed(3)
        v0 = torch.rand((B, C_out, H, W), generator=g) * 0.4
        rep2, _, r2, v_fin = run_case(dev, case, neuron="if", v_th=0.5, v_reset=0.0, v0=v0, traces=traces)
        assert rep2.ok, str(rep2)
        assert torch.allclose(v_fin, r2.v_final, rtol=1e-3, atol=1e-3)
    finally:
        ops.set_fused_kernel("auto")
        del os.environ["SENGINE_AMD_TILE_KSPLIT"]
        del os.environ["SENGINE_AMD_TILE_SHAPE"]


@pytest.mark.parametrize("traces", [True, False])
@pytest.mark.parametrize("pf", ["1", "2"])
@pytest.mark.parametrize("ksplit,shape", [("1", "0"), ("1", "1"), ("1", "2"), ("2", "2")])
@pytest.mark.parametrize("H,W,C_in,C_out,B", [(7, 7, 256, 128, 3), (13, 11, 192, 64, 2), (14, 14, 128, 128, 1)])
def test_tile_prefetch_depth(dev, pf, ksplit, shape, H, W, C_in, C_out, B, traces):
    """3x3 halo tiles with one- and two-deep operand prefetch (SENGINE_AMD_TILE_PF): A operands
    fetched across the 64-channel chunk boundary, B fragments two steps ahead; odd and even
    chunk counts, ragged tiles, LIF fast epilogue and IF with state, against the oracle."""
    import os
    if ksplit == "2" and (C_in // 64) % 2:
        pytest.skip("the reduction split needs an even number of 64-channel chunks")
    os.environ["SENGINE_AMD_TILE_PF"] = pf
    os.environ["SENGINE_AMD_TILE_KSPLIT"] = ksplit
    os.environ["SENGINE_AMD_TILE_SHAPE"] = shape
    ops.set_fused_kernel("tile")  # small test shapes would otherwise take the small-M kernel
    try:
        case = ref.make_layer_case(130 + H + C_in // 64, T=4, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=3,
                                   fp16_weights=True, p_spike=0.2)
        rep, x_err, _, _ = run_case(dev, case, traces=traces)
        assert rep.ok, str(rep)
        assert x_err is None or x_err < 1e-4
        g = torch.Generator().manual_seed(4)
        v0 = torch.rand((B, C_out, H, W), generator=g) * 0.4
        rep2, _, r2, v_fin = run_case(dev, case, neuron="if", v_th=0.5, v_reset=0.0, v0=v0, traces=traces)
        assert rep2.ok, str(rep2)
        assert torch.allclose(v_fin, r2.v_final, rtol=1e-3, atol=1e-3)
    finally:
        ops.set_fused_kernel("auto")
        for k in ("SENGINE_AMD_TILE_PF", "SENGINE_AMD_TILE_KSPLIT", "SENGINE_AMD_TILE_SHAPE"):
            del os.environ[k]


# ---- flat small-output layout: <= 16 output pixels per image run as one GEMM per image
# flat: (2,2,3,1,1) (3,3,3,2,1) (2,3,3,1,1) (2,2,3,2,1) (1,2,1,2,0) (3,2,3,2,1); the rest
# have small outputs on inputs over 2x the kernel window or whose flat matrix would hold over
# 4x the conv's weights, so they take the small-M kernel on the ordinary layout
FLAT_CASES = [(2, 2, 3, 1, 1, 256, 256, 5, 4), (3, 3, 3, 2, 1, 64, 128, 2, 4), (2, 3, 3, 1, 1, 128, 128, 3, 8),
              (2, 2, 3, 2, 1, 256, 512, 4, 1), (1, 2, 1, 2, 0, 64, 128, 3, 4), (3, 2, 3, 2, 1, 64, 64, 2, 4),
              (4, 4, 3, 2, 1, 128, 256, 3, 4), (4, 4, 3, 1, 1, 128, 128, 3, 8),
              (6, 6, 3, 2, 1, 64, 128, 2, 2), (2, 2, 1, 2, 0, 64, 128, 3, 4), (5, 3, 3, 2, 1, 64, 64, 2, 4)]


@pytest.mark.parametrize("kernel", ["auto", "direct"])
@pytest.mark.parametrize("H,W,k,stride,pad,C_in,C_out,B,T", FLAT_CASES)
def test_flat_layout_against_oracle(dev, kernel, H, W, k, stride, pad, C_in, C_out, B, T):
    """Small outputs (flat layout where it applies): the split-K small-M kernel ('auto') and
    the direct kernel, with traces, against the oracle."""
    ops.set_fused_kernel(kernel)
    try:
        case = ref.make_layer_case(60 + H + k + C_in // 64, T=T, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=k,
                                   stride=stride, padding=pad, fp16_weights=True, p_spike=0.3)
        rep, x_err, r, _ = run_case(dev, case)
        print(rep, x_err, float(r.spikes.mean()))
        assert rep.ok, str(rep)
        assert x_err < 1e-4
        assert float(r.spikes.mean()) > 0.001
    finally:
        ops.set_fused_kernel("auto")


@pytest.mark.parametrize("in_enc,out_enc,planes", [(ops.ENC_BITS, ops.ENC_F16, 1), (ops.ENC_F16, ops.ENC_BITS, 1),
                                                   (ops.ENC_F16, ops.ENC_F16, 2), (ops.ENC_BITS, ops.ENC_BITS, 2)])
@pytest.mark.parametrize("H", [2, 4])
def test_flat_layout_encodings_and_state(dev, in_enc, out_enc, planes, H):
    """Encodings, two weight planes and a carried membrane on a flat layer (2x2) and on a
    small non-flat one (4x4)."""
    case = ref.make_layer_case(71 + H, T=4, B=3, C_in=128, C_out=128, H=H, W=H, k=3, stride=1, padding=1,
                               fp16_weights=(planes == 1), p_spike=0.3)
    g = torch.Generator().manual_seed(6)
    v0 = torch.rand((3, 128, H, H), generator=g) * 0.9
    rep, x_err, r, v_fin = run_case(dev, case, planes=planes, in_enc=in_enc, out_enc=out_enc, v0=v0)
    assert rep.ok, str(rep)
    assert torch.allclose(v_fin, r.v_final, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("H,W,k,stride,pad,flat", [(2, 2, 3, 1, 1, True), (3, 3, 3, 2, 1, True),
                                                    (1, 2, 1, 2, 0, True), (3, 2, 3, 2, 1, True),
                                                    (4, 4, 3, 1, 1, False), (6, 6, 3, 2, 1, False),
                                                    (3, 4, 3, 2, 1, False), (2, 2, 1, 2, 0, False)])
def test_flat_compressor_matches_numpy(dev, H, W, k, stride, pad, flat):
    """The compressor emits the flat blob for small outputs whose flat matrix stays within 4x
    the conv's weight entries and whose input is at most 2x the kernel window: byte-identical
    to the numpy restatement applied to oracle.packing.flat_weight; other small outputs keep
    the ordinary layout."""
    g = torch.Generator().manual_seed(H * W + k)
    w = ref.prune_conv_2_4(torch.randn((128, 64, k, k), generator=g) * 0.05).half().float()
    spec = ops.ConvSpec(T=4, B=2, C_in=64, H=H, W=W, C_out=128, KH=k, KW=k, stride=stride, padding=pad)
    values, meta, viol = ops.compress_2_4(spec, w.to(dev))
    wl = pk.flat_weight(w.numpy(), H, W, stride, pad) if flat else w.numpy()
    ev, em, _ = pk.compress_2_4(wl, 1)
    assert np.array_equal(values.cpu().numpy().view(np.uint16), ev.reshape(-1))
    assert np.array_equal(meta.cpu().numpy().view(np.uint32), em.reshape(-1))
    assert int(viol.sum()) == 0


@pytest.mark.parametrize("traces", [True, False])
@pytest.mark.parametrize("pm", ["1", "2"])
@pytest.mark.parametrize("C_in,C_out,H,W,stride,B", [(256, 512, 7, 9, 1, 3), (128, 1024, 6, 5, 1, 2),
                                                     (384, 512, 9, 10, 2, 2), (512, 256, 4, 13, 1, 2)])
def test_tile1_position_major(dev, pm, C_in, C_out, H, W, stride, B, traces):
    """1x1 convs on the position-major kernel (tile1pm.h: 16 positions x 4 waves of 64*GPW
    channels per workgroup, 2 or 4 chunks per staging phase) with GPW forced to 1 or 2, ragged
    position counts, stride 2, LIF (fast or generic epilogue) and IF with a carried membrane."""
    import os
    if pm == "2" and C_out % 512:
        pytest.skip("two channel groups per wave need C_out % 512 == 0")
    os.environ["SENGINE_AMD_TILE1_PM"] = pm
    ops.set_fused_kernel("tile")  # small test shapes would otherwise take the small-M kernel
    try:
        case = ref.make_layer_case(150 + C_in // 64 + C_out // 64 + stride, T=4, B=B, C_in=C_in, C_out=C_out, H=H,
                                   W=W, k=1, stride=stride, padding=0, fp16_weights=True, p_spike=0.2)
        spec = ops.ConvSpec(T=4, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=1, KW=1, stride=stride, padding=0)
        plan = ops.fused_plan(spec, traces=traces)
        assert plan.startswith(f"tile1pm<T=4,GPW={pm},"), plan
        rep, x_err, _, _ = run_case(dev, case, traces=traces)
        assert rep.ok, str(rep)
        assert x_err is None or x_err < 1e-4
        g = torch.Generator().manual_seed(5)
        OH = (H - 1) // stride + 1
        OW = (W - 1) // stride + 1
        v0 = torch.rand((B, C_out, OH, OW), generator=g) * 0.4
        rep2, _, r2, v_fin = run_case(dev, case, neuron="if", v_th=0.5, v_reset=0.0, v0=v0, traces=traces)
        assert rep2.ok, str(rep2)
        assert torch.allclose(v_fin, r2.v_final, rtol=1e-3, atol=1e-3)
    finally:
        ops.set_fused_kernel("auto")
        del os.environ["SENGINE_AMD_TILE1_PM"]



F16_TILE_CASES = [(3, 1, "0", 13, 11, 128, 64, 2), (3, 1, "1", 16, 9, 64, 128, 1), (3, 1, "2", 7, 7, 192, 64, 3),
                  (1, 1, None, 7, 9, 256, 128, 3), (1, 2, None, 11, 10, 128, 192, 2)]


@pytest.mark.parametrize("state", [False, True])
@pytest.mark.parametrize("out_enc", [ops.ENC_BITS, ops.ENC_F16])
@pytest.mark.parametrize("C,H,W,B,shape", [(256, 7, 7, 4, "2"), (128, 16, 16, 2, "0"), (128, 14, 8, 2, "1")])
def test_tile_f16_input_reduction_split(dev, env, C, H, W, B, shape, out_enc, state):
    """fp16-input 3x3 layers on grids of at most one workgroup per CU (the exported per-node
    call's 7x7 layer) split the reduction over two wave sets: each tile shape, both outputs,
    with and without the membrane state, against the oracle and identical to the unsplit kernel."""
    env("SENGINE_AMD_TILE_SHAPE", shape)
    spec = ops.ConvSpec(T=4, B=B, C_in=C, H=H, W=W, C_out=C, KH=3, KW=3, stride=1, padding=1,
                        in_enc=ops.ENC_F16, out_enc=out_enc)
    ops.set_fused_kernel("tile")  # small shapes would otherwise take the small-M kernel
    try:
        plan = ops.fused_plan(spec, state=state)
        assert plan.startswith("tile<T=4,KS=3,") and ",KSP=2," in plan and "in=f16" in plan, plan
        case = ref.make_layer_case(380 + C // 64 + H, T=4, B=B, C_in=C, C_out=C, H=H, W=W, k=3, padding=1,
                                   fp16_weights=True, p_spike=0.2)
        v0 = torch.rand((B, C, H, W), generator=torch.Generator().manual_seed(9)) * 0.4 if state else None
        rep, _, r, v_fin = run_case(dev, case, in_enc=ops.ENC_F16, out_enc=out_enc, v0=v0, traces=False)
        assert rep.ok, str(rep)
        if state:
            assert torch.allclose(v_fin, r.v_final, rtol=1e-3, atol=1e-3)
        env("SENGINE_AMD_TILE_KSPLIT", 1)
        assert ",KSP=1," in ops.fused_plan(spec, state=state)
        rep1, _, _, v_fin1 = run_case(dev, case, in_enc=ops.ENC_F16, out_enc=out_enc, v0=v0, traces=False)
        assert rep1.ok, str(rep1)
        if state:
            assert torch.allclose(v_fin, v_fin1, rtol=1e-5, atol=1e-6)
    finally:
        ops.set_fused_kernel("auto")


@pytest.mark.parametrize("traces", [True, False])
@pytest.mark.parametrize("out_enc", [ops.ENC_BITS, ops.ENC_F16])
@pytest.mark.parametrize("k,stride,shape,H,W,C_in,C_out,B", F16_TILE_CASES)
def test_tile_f16_input(dev, k, stride, shape, H, W, C_in, C_out, B, out_enc, traces):
    """fp16 NHWC activations (the reference's call() ABI) through the tile kernels: each 3x3
    halo-tile shape and 1x1 at stride 1 and 2, bit and fp16 output, LIF with hard reset (fast
    epilogue), IF with a carried membrane and LIF with soft reset (generic epilogue)."""
    import os
    if shape is not None:
        os.environ["SENGINE_AMD_TILE_SHAPE"] = shape
    ops.set_fused_kernel("tile")  # small test shapes would otherwise take the small-M kernel
    try:
        spec = ops.ConvSpec(T=4, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=k, KW=k, stride=stride, padding=k // 2,
                            in_enc=ops.ENC_F16, out_enc=out_enc)
        plan = ops.fused_plan(spec, traces=traces)
        assert plan.startswith(f"tile<T=4,KS={k},") and "in=f16" in plan, plan
        case = ref.make_layer_case(170 + k + stride + C_in // 64, T=4, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=k,
                                   stride=stride, padding=k // 2, fp16_weights=True, p_spike=0.2)
        rep, x_err, _, _ = run_case(dev, case, in_enc=ops.ENC_F16, out_enc=out_enc, traces=traces)
        assert rep.ok, str(rep)
        assert x_err is None or x_err < 1e-4
        OH, OW = (H - 1) // stride + 1, (W - 1) // stride + 1
        g = torch.Generator().manual_seed(7)
        v0 = torch.rand((B, C_out, OH, OW), generator=g) * 0.4
        rep2, _, r2, v_fin = run_case(dev, case, neuron="if", v_th=0.5, v_reset=0.0, v0=v0, in_enc=ops.ENC_F16,
                                      out_enc=out_enc, traces=traces)
        assert rep2.ok, str(rep2)
        assert torch.allclose(v_fin, r2.v_final, rtol=1e-3, atol=1e-3)
        rep3, _, _, _ = run_case(dev, case, v_th=0.5, v_reset=None, in_enc=ops.ENC_F16, out_enc=out_enc,
                                 traces=traces)
        assert rep3.ok, str(rep3)
    finally:
        ops.set_fused_kernel("auto")
        os.environ.pop("SENGINE_AMD_TILE_SHAPE", None)


@pytest.mark.parametrize("k", [3, 1])
def test_tile_f16_input_real_valued(dev, k):
    """Any fp16 activation, not only 0/1 spikes: fp16 values in [-2, 2) (exact in fp16) on the
    fp16-input tile kernel; sums of exact fp16 products in fp32 agree with the fp32 oracle
    within the membrane tolerance, spikes by the flip rule."""
    case = ref.make_layer_case(190 + k, T=4, B=2, C_in=128, C_out=128, H=10, W=9, k=k, fp16_weights=True)
    g = torch.Generator().manual_seed(11)
    x = (torch.rand(case.x_seq.shape, generator=g) * 4 - 2).half().float()
    case = ref.LayerCase(x * (torch.rand(x.shape, generator=g) < 0.5), case.w, case.bn, case.stride, case.padding)
    ops.set_fused_kernel("tile")
    try:
        spec = ops.ConvSpec(T=4, B=2, C_in=128, H=10, W=9, C_out=128, KH=k, KW=k, stride=1, padding=k // 2,
                            in_enc=ops.ENC_F16)
        assert "in=f16" in ops.fused_plan(spec)
        rep, x_err, r, _ = run_case(dev, case, in_enc=ops.ENC_F16)
        print(rep, x_err, float(r.spikes.mean()))
        assert rep.ok, str(rep)
        assert x_err < 1e-3
    finally:
        ops.set_fused_kernel("auto")


@pytest.mark.parametrize("traces", [True, False])
@pytest.mark.parametrize("out_enc", [ops.ENC_BITS, ops.ENC_F16])
@pytest.mark.parametrize("C_in,C_out,H,W,stride,B", [(384, 384, 7, 9, 1, 3), (128, 768, 6, 5, 1, 2),
                                                     (256, 256, 9, 10, 2, 2), (128, 512, 4, 13, 1, 1)])
def test_tile1pm_f16_input(dev, C_in, C_out, H, W, stride, B, out_enc, traces):
    """fp16 activations on the position-major 1x1 kernel (6 waves for 384-channel multiples,
    else 4; phases of two chunks), ragged position counts, stride 2, bit and fp16 output, LIF
    (fast or generic epilogue) and IF with a carried membrane, against the oracle."""
    spec = ops.ConvSpec(T=4, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=1, KW=1, stride=stride, padding=0,
                        in_enc=ops.ENC_F16, out_enc=out_enc)
    plan = ops.fused_plan(spec, traces=traces)
    nw = 6 if C_out % 384 == 0 else 4
    assert plan.startswith(f"tile1pm<T=4,GPW=1,CG=2,NW={nw},in=f16,"), plan
    case = ref.make_layer_case(230 + C_in // 64 + C_out // 64 + stride, T=4, B=B, C_in=C_in, C_out=C_out, H=H, W=W,
                               k=1, stride=stride, padding=0, fp16_weights=True, p_spike=0.2)
    rep, x_err, _, _ = run_case(dev, case, in_enc=ops.ENC_F16, out_enc=out_enc, traces=traces)
    assert rep.ok, str(rep)
    assert x_err is None or x_err < 1e-4
    g = torch.Generator().manual_seed(6)
    OH, OW = (H - 1) // stride + 1, (W - 1) // stride + 1
    v0 = torch.rand((B, C_out, OH, OW), generator=g) * 0.4
    rep2, _, r2, v_fin = run_case(dev, case, neuron="if", v_th=0.5, v_reset=0.0, v0=v0, in_enc=ops.ENC_F16,
                                  out_enc=out_enc, traces=traces)
    assert rep2.ok, str(rep2)
    assert torch.allclose(v_fin, r2.v_final, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("neuron", ["lif", "if"])
@pytest.mark.parametrize("shape,C_in,C_out,H,W,B,slots", [("0", 64, 64, 13, 11, 2, 5), ("1", 128, 128, 15, 9, 3, 8),
                                                         ("2", 192, 64, 7, 7, 4, 3), ("0", 64, 192, 17, 8, 2, 7)])
def test_tile3ps_walks(dev, shape, C_in, C_out, H, W, B, slots, neuron):
    """The persistent 3x3 kernel (tile3ps.h), forced onto small layers (SENGINE_AMD_TILE3_PS=2)
    with few resident workgroups (SENGINE_AMD_PS_SLOTS) so each walks several ragged tiles: one,
    two and three reduction chunks, one and three channel blocks, every tile shape, LIF and IF,
    against the oracle."""
    os.environ.update(SENGINE_AMD_TILE3_PS="2", SENGINE_AMD_PS_SLOTS=str(slots), SENGINE_AMD_TILE_SHAPE=shape,
                      SENGINE_AMD_TILE_PF="1", SENGINE_AMD_TILE_KSPLIT="1")
    ops.set_fused_kernel("tile")
    try:
        spec = ops.ConvSpec(T=4, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=3, KW=3, stride=1, padding=1,
                            neuron=neuron)
        plan = ops.fused_plan(spec)
        assert plan.startswith("tile3ps<T=4,"), plan
        print(plan)
        case = ref.make_layer_case(280 + C_in // 64 + C_out // 64 + H, T=4, B=B, C_in=C_in, C_out=C_out, H=H, W=W,
                                   k=3, fp16_weights=True, p_spike=0.25)
        kw = dict(neuron="if", v_th=0.5, v_reset=0.0) if neuron == "if" else {}
        rep, _, r, _ = run_case(dev, case, traces=False, **kw)
        print(rep, float(r.spikes.mean()))
        assert rep.ok, str(rep)
        assert float(r.spikes.mean()) > 0.002
    finally:
        for k in ("SENGINE_AMD_TILE3_PS", "SENGINE_AMD_PS_SLOTS", "SENGINE_AMD_TILE_SHAPE", "SENGINE_AMD_TILE_PF",
                  "SENGINE_AMD_TILE_KSPLIT"):
            os.environ.pop(k, None)
        ops.set_fused_kernel("auto")


@pytest.mark.parametrize("slots", [0, 3])
@pytest.mark.parametrize("neuron", ["lif", "if"])
@pytest.mark.parametrize("C_in,C_out,H,W,B", [(384, 512, 64, 40, 2), (128, 1024, 8, 16, 2), (128, 256, 4, 4, 1),
                                             (384, 384, 64, 40, 2), (384, 1152, 4, 8, 1)])
@pytest.mark.parametrize("out_enc", ["bits", "f16"])
def test_tile1ps_f16_input(dev, C_in, C_out, H, W, B, neuron, slots, out_enc):
    """The persistent fp16-input 1x1 kernel (token Linears: stride 1, 16 | M, spike bits out;
    the exported per-node call's fp16 spikes out; stateless hard-reset neuron): 4-wave
    super-blocks with resident workgroups walking 1 or 2 position groups each (5,120 positions
    over 256 workgroups per super-block), a single group, four super-blocks; 6-wave 384-channel
    super-blocks (phases of three chunks), one per CU walking 1 or 2 groups, or three
    super-blocks; LIF and IF, against the oracle.  The direct-staged kernel (tile1ds.h), which
    takes 4- and 6-chunk layers of 256 | C_out by default, is switched off here; it has its own
    tests (tests/test_gpu_tile1ds.py)."""
    if slots:  # few resident workgroups: every one walks many groups
        os.environ["SENGINE_AMD_PS_SLOTS"] = str(slots)
    os.environ["SENGINE_AMD_TILE1_DS"] = "0"
    try:
        spec = ops.ConvSpec(T=4, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=1, KW=1, stride=1, padding=0,
                            neuron=neuron, in_enc=ops.ENC_F16,
                            out_enc=ops.ENC_F16 if out_enc == "f16" else ops.ENC_BITS)
        plan = ops.fused_plan(spec)
        nw, cg = (4, 2) if C_out % 256 == 0 else (6, 3)
        assert plan.startswith(f"tile1ps<T=4,NW={nw},CG={cg},in=f16,out={out_enc},"), plan
        print(plan)
        case = ref.make_layer_case(260 + C_in // 64 + C_out // 64, T=4, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=1,
                                   padding=0, fp16_weights=True, p_spike=0.2)
        kw = dict(neuron="if", v_th=0.5, v_reset=0.0) if neuron == "if" else {}
        rep, _, r, _ = run_case(dev, case, in_enc=ops.ENC_F16, out_enc=spec.out_enc, traces=False, **kw)
        print(rep, float(r.spikes.mean()))
        assert rep.ok, str(rep)
        assert float(r.spikes.mean()) > 0.002  # the comparison covers firing neurons
    finally:
        os.environ.pop("SENGINE_AMD_PS_SLOTS", None)
        os.environ.pop("SENGINE_AMD_TILE1_DS", None)


@pytest.mark.parametrize("npg", [1, 2])
@pytest.mark.parametrize("C_in,C_out,H,W,B,mode", [(768, 384, 64, 40, 2, "res16"), (256, 512, 32, 32, 2, "f16"),
                                                    (384, 384, 48, 32, 1, "res16"), (256, 1024, 16, 16, 2, "bits"),
                                                    (1536, 384, 28, 52, 1, "res16"), (384, 384, 32, 48, 1, "bits")])
def test_tile1ps_bits_input(dev, C_in, C_out, H, W, B, mode, npg):
    """The persistent 1x1 kernel on spike bits (the token Linears fed by spikes: proj, fc2):
    fp16 spikes + the fp16 residual stream out (6-wave 384-channel super-blocks: 32-position
    groups with phases of three chunks, or with SENGINE_AMD_TILE1_NPG=1 -- and always when
    32 does not divide M -- 16-position groups with phases of six; one workgroup per CU walking
    a few of hundreds of groups, or one group each), plain fp16 spikes (4-wave super-blocks,
    phases of four chunks), and spike bits out (the opt-in SENGINE_AMD_TILE1_PS=2), against the
    oracle."""
    T = 4
    out_enc = ops.ENC_BITS if mode == "bits" else ops.ENC_F16
    spec = ops.ConvSpec(T=T, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=1, KW=1, stride=1, padding=0,
                        out_enc=out_enc)
    if mode == "bits":
        os.environ["SENGINE_AMD_TILE1_PS"] = "2"
    os.environ["SENGINE_AMD_TILE1_NPG"] = str(npg)
    try:
        plan = ops.fused_plan(spec)
        pos32 = C_out % 384 == 0 and npg == 2 and (B * H * W) % 32 == 0
        nw, cg = ((6, 3) if pos32 else (6, 6)) if C_out % 384 == 0 else (4, 4)
        assert plan.startswith(f"tile1ps<T=4,NW={nw},CG={cg},in=bits,out={'bits' if mode == 'bits' else 'f16'},"), plan
        assert (",pos=32>" in plan) == pos32, plan
        print(plan)
        case = ref.make_layer_case(270 + C_in // 64 + C_out // 64, T=T, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=1,
                                   padding=0, fp16_weights=True, p_spike=0.15)
        values, meta, _ = ops.compress_2_4(spec, case.w.to(dev))
        sc, bi = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
        sc_d, bi_d = torch.from_numpy(sc).to(dev), torch.from_numpy(bi).to(dev)
        data = torch.from_numpy(pk.seq_to_nhwc_bits(case.x_seq.numpy()).view(np.int32)).to(dev)
        r = ref.fused_layer(case.x_seq, case.w, case.bn, 1, 0, 1, "lif", 2.0, 1.0, 0.0)
        if mode == "res16":
            g = torch.Generator().manual_seed(C_out)
            res_int = torch.randint(0, 18, (T * B, H, W, C_out), generator=g)
            out = ops.fused_sparse_conv_bn_lif_add(spec, data, values, meta, sc_d, bi_d, res_int.half().to(dev), 0, 0)
            torch.cuda.synchronize()
            spk = out.float().cpu() - res_int.float()
        else:
            out = ops.fused_sparse_conv_bn_lif(spec, data, values, meta, sc_d, bi_d)
            torch.cuda.synchronize()
            if mode == "bits":
                spk = torch.from_numpy(pk.unpack_bits(out.cpu().numpy().view(np.uint32).reshape(-1, C_out // 32),
                                                      C_out).reshape(T * B, H, W, C_out)).float()
            else:
                spk = out.float().cpu()
        assert set(np.unique(spk.numpy())) <= {0.0, 1.0}
        rep = compare(nhwc_seq(spk, T), None, r.spikes.numpy(), r.h.numpy(), 1.0)
        print(rep, float(r.spikes.mean()))
        assert rep.ok, str(rep)
        assert float(r.spikes.mean()) > 0.002
    finally:
        os.environ.pop("SENGINE_AMD_TILE1_PS", None)
        os.environ.pop("SENGINE_AMD_TILE1_NPG", None)


@pytest.mark.parametrize("slots", [1, 3, 5])
def test_tile1ps_pos32_walks_many_groups(dev, slots):
    """32-position groups on a few resident workgroups, each walking dozens of groups (the
    A-operand ring and the phase buffers wrap many times, across group boundaries): spikes and
    the fp16 stream identical to the 16-position-group kernel's."""
    T, B, C_in, C_out, H, W = 4, 1, 1536, 384, 64, 40
    spec = ops.ConvSpec(T=T, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=1, KW=1, stride=1, padding=0,
                        out_enc=ops.ENC_F16)
    case = ref.make_layer_case(290 + slots, T=T, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=1, padding=0,
                               fp16_weights=True, p_spike=0.15)
    values, meta, _ = ops.compress_2_4(spec, case.w.to(dev))
    sc, bi = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
    sc_d, bi_d = torch.from_numpy(sc).to(dev), torch.from_numpy(bi).to(dev)
    data = torch.from_numpy(pk.seq_to_nhwc_bits(case.x_seq.numpy()).view(np.int32)).to(dev)
    res = torch.randint(0, 18, (T * B, H, W, C_out), generator=torch.Generator().manual_seed(slots)).half().to(dev)
    outs = []
    try:
        os.environ["SENGINE_AMD_PS_SLOTS"] = str(slots)
        for npg in (2, 1):
            os.environ["SENGINE_AMD_TILE1_NPG"] = str(npg)
            plan = ops.fused_plan(spec)
            assert (",pos=32>" in plan) == (npg == 2), plan
            outs.append(ops.fused_sparse_conv_bn_lif_add(spec, data, values, meta, sc_d, bi_d, res, 0, 0))
        torch.cuda.synchronize()
    finally:
        os.environ.pop("SENGINE_AMD_PS_SLOTS", None)
        os.environ.pop("SENGINE_AMD_TILE1_NPG", None)
    assert torch.equal(outs[0], outs[1])
    r = ref.fused_layer(case.x_seq, case.w, case.bn, 1, 0, 1, "lif", 2.0, 1.0, 0.0)
    spk = outs[0].float().cpu() - res.float().cpu()
    rep = compare(nhwc_seq(spk, T), None, r.spikes.numpy(), r.h.numpy(), 1.0)
    assert rep.ok, str(rep)


@pytest.mark.parametrize("res", ["none", "f16", "bits"])
@pytest.mark.parametrize("C,H,W,B", [(64, 56, 56, 4), (128, 28, 28, 8), (256, 14, 14, 16), (384, 14, 14, 8)])
def test_tile3_f16_output_fast_epilogue(dev, C, H, W, B, res):
    """3x3 spike-bit convolutions writing fp16 spikes (a transformer stem's last conv, whose
    spikes start the fp16 residual stream) run the fast hard-reset epilogue, alone and adding an
    fp16 residual of integers or a one-plane spike-bit residual (Spikformer's rpe conv plus the
    pooled patch features), on every tile shape, against the oracle."""
    T = 4
    spec = ops.ConvSpec(T=T, B=B, C_in=C, H=H, W=W, C_out=C, KH=3, KW=3, stride=1, padding=1, out_enc=ops.ENC_F16)
    plan = ops.fused_plan(spec)
    assert plan.startswith("tile<T=4,KS=3,") and "out=f16,epi=lif_hard" in plan, plan
    print(plan)
    case = ref.make_layer_case(330 + C // 64 + H, T=T, B=B, C_in=C, C_out=C, H=H, W=W, k=3, padding=1,
                               fp16_weights=True, p_spike=0.2)
    values, meta, _ = ops.compress_2_4(spec, case.w.to(dev))
    sc, bi = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
    sc_d, bi_d = torch.from_numpy(sc).to(dev), torch.from_numpy(bi).to(dev)
    data = torch.from_numpy(pk.seq_to_nhwc_bits(case.x_seq.numpy()).view(np.int32)).to(dev)
    r = ref.fused_layer(case.x_seq, case.w, case.bn, 1, 1, 1, "lif", 2.0, 1.0, 0.0)
    if res == "f16":
        res_int = torch.randint(0, 6, (T * B, H, W, C), generator=torch.Generator().manual_seed(C + H))
        out = ops.fused_sparse_conv_bn_lif_add(spec, data, values, meta, sc_d, bi_d, res_int.half().to(dev), 0, 0)
        torch.cuda.synchronize()
        spk = out.float().cpu() - res_int.float()
    elif res == "bits":
        res_int = (torch.rand((T * B, H, W, C), generator=torch.Generator().manual_seed(C + W)) < 0.3).half()
        out = ops.fused_sparse_conv_bn_lif_add(spec, data, values, meta, sc_d, bi_d,
                                               ops.pack_spikes(res_int.to(dev)), 1, 0)
        torch.cuda.synchronize()
        spk = out.float().cpu() - res_int.float()
    else:
        out = ops.fused_sparse_conv_bn_lif(spec, data, values, meta, sc_d, bi_d)
        torch.cuda.synchronize()
        spk = out.float().cpu()
    assert set(np.unique(spk.numpy())) <= {0.0, 1.0}
    rep = compare(nhwc_seq(spk, T), None, r.spikes.numpy(), r.h.numpy(), 1.0)
    print(rep, float(r.spikes.mean()))
    assert rep.ok, str(rep)
    assert float(r.spikes.mean()) > 0.002


@pytest.mark.parametrize("C_out", [384, 128])
def test_fp16_residual_stream_add(dev, C_out):
    """out = spike + residual as fp16 (the reference add kernel's form) with an fp16 residual
    and with a one-plane bit residual, against the oracle's spikes plus the residual; the
    residual holds integers up to 17 (Spikformer's stream after eight blocks)."""
    T, B, C_in, H, W = 4, 2, 128, 6, 7
    case = ref.make_layer_case(250 + C_out // 64, T=T, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=1, padding=0,
                               fp16_weights=True, p_spike=0.3)
    spec = ops.ConvSpec(T=T, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=1, KW=1, stride=1, padding=0,
                        out_enc=ops.ENC_F16)
    values, meta, _ = ops.compress_2_4(spec, case.w.to(dev))
    sc, bi = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
    sc_d, bi_d = torch.from_numpy(sc).to(dev), torch.from_numpy(bi).to(dev)
    data = torch.from_numpy(pk.seq_to_nhwc_bits(case.x_seq.numpy()).view(np.int32)).to(dev)
    r = ref.fused_layer(case.x_seq, case.w, case.bn, 1, 0, 1, "lif", 2.0, 1.0, 0.0)
    s_ref = r.spikes.numpy()  # (T, B, C_out, H, W)
    g = torch.Generator().manual_seed(C_out)
    res_int = torch.randint(0, 18, (T * B, H, W, C_out), generator=g)
    out = ops.fused_sparse_conv_bn_lif_add(spec, data, values, meta, sc_d, bi_d, res_int.half().to(dev), 0, 0)
    torch.cuda.synchronize()
    spk = out.float().cpu() - res_int.float()
    rep = compare(nhwc_seq(spk, T), None, s_ref, r.h.numpy(), 1.0)
    assert rep.ok, str(rep)
    assert set(np.unique(spk.numpy())) <= {0.0, 1.0}
    # one-plane bit residual (the spikes of another layer), fp16 output
    res_bits = (torch.rand((T * B, H, W, C_out), generator=g) < 0.4).half()
    out2 = ops.fused_sparse_conv_bn_lif_add(spec, data, values, meta, sc_d, bi_d, ops.pack_spikes(res_bits.to(dev)),
                                            1, 0)
    torch.cuda.synchronize()
    assert torch.equal(out2.float().cpu() - res_bits.float(), spk)


@pytest.mark.parametrize("C_in,C_out,split,H,W,B,in_enc", [(384, 1280, 384, 64, 40, 2, "f16"), (128, 512, 128, 16, 8, 2, "f16"),
                                                         (128, 384, 128, 16, 16, 2, "bits"),
                                                         (64, 192, 64, 9, 7, 2, "bits"),
                                                         (64, 128, 64, 16, 16, 2, "bits")])
def test_fused_split_output(dev, C_in, C_out, split, H, W, B, in_enc, monkeypatch):
    """The channel-split spike output (sengine_amd_fused_sparse_conv_bn_lif_split: channel c
    in plane c / split): equal, plane by plane, to the plain call's bits, for the persistent
    fp16-input 1x1 kernel (Spikformer's concatenated q/k/v, padded to 1280 channels), another
    1x1 route and 3x3 layers (the 16x16 one with the persistent 3x3 kernel forced where it is
    eligible, which a split output must make it not be), and the plain call is against the
    oracle."""
    k = 3 if C_in == 64 else 1
    if H == 16 and k == 3:
        monkeypatch.setenv("SENGINE_AMD_TILE3_PS", "2")
    f16 = in_enc == "f16"
    spec = ops.ConvSpec(T=4, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=k, KW=k, stride=1, padding=k // 2,
                        in_enc=ops.ENC_F16 if f16 else ops.ENC_BITS)
    case = ref.make_layer_case(330 + C_out // 64, T=4, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=k, padding=k // 2,
                               fp16_weights=True, p_spike=0.2)
    rep, _, _, _ = run_case(dev, case, in_enc=spec.in_enc, traces=False)
    assert rep.ok, str(rep)
    values, meta, _ = ops.compress_2_4(spec, case.w.to(dev))
    sc, bi = ref.fold_batchnorm(case.bn.gamma, case.bn.beta, case.bn.mean, case.bn.var, case.bn.eps)
    sc_d, bi_d = torch.from_numpy(sc).to(dev), torch.from_numpy(bi).to(dev)
    T = 4
    if f16:
        data = case.x_seq.permute(0, 1, 3, 4, 2).reshape(T * B, H, W, C_in).contiguous().half().to(dev)
    else:
        data = torch.from_numpy(pk.seq_to_nhwc_bits(case.x_seq.numpy()).view(np.int32)).to(dev)
    plain = ops.fused_sparse_conv_bn_lif(spec, data, values, meta, sc_d, bi_d)
    planes = ops.fused_sparse_conv_bn_lif_split(spec, data, values, meta, sc_d, bi_d, split)
    torch.cuda.synchronize()
    print(ops.fused_plan(spec), tuple(planes.shape))
    full = plain.view(T * B * H * W, C_out // 32)
    for j in range(-(-C_out // split)):
        n = min(split, C_out - j * split) // 32
        assert torch.equal(planes[j].reshape(T * B * H * W, split // 32)[:, :n], full[:, j * split // 32:j * split // 32 + n])


def _tail_case(seed, B, C_in, C_out, H, W, p_spike=0.2):
    """A 3x3 layer whose last 32 input channels are padding: zero weights there (the input
    spikes in those channels stay random: the paired-tail call must not depend on them)."""
    case = ref.make_layer_case(seed, T=4, B=B, C_in=C_in, C_out=C_out, H=H, W=W, k=3, padding=1,
                               fp16_weights=True, p_spike=p_spike)
    case.w[:, C_in - 32:] = 0.0
    return case


@pytest.mark.gpu
@pytest.mark.parametrize("neuron", ["lif", "if"])
@pytest.mark.parametrize("state", [False, True])
@pytest.mark.parametrize("shape", ["0", "1", "2"])
@pytest.mark.parametrize("C_in,C_out,H,W,B", [(128, 64, 16, 16, 2), (64, 128, 13, 11, 3), (192, 64, 14, 9, 2)])
def test_tail_pairs_taps(dev, env, C_in, C_out, H, W, B, shape, state, neuron):
    """The paired-tail call (the last chunk's 32 real channels of two taps per reduction step) on
    every tile shape, one to three channel chunks, ragged images, both neurons, with and without
    the membrane state, against the oracle of the padded conv; and the same spikes as the
    ordinary call on the padded blob up to the parity rule."""
    env("SENGINE_AMD_TILE_SHAPE", shape)
    case = _tail_case(400 + C_in + H + int(shape), B, C_in, C_out, H, W)
    spec = ops.ConvSpec(T=4, B=B, C_in=C_in, H=H, W=W, C_out=C_out, KH=3, KW=3, stride=1, padding=1,
                        neuron=neuron, hard_reset=True, tau=2.0, v_threshold=1.0, v_reset=0.0)
    plan = ops.fused_plan(spec, state=state, tail=True)
    assert plan.startswith("tile3ps<") and ",pair>" in plan and f"{9 * (C_in // 64 - 1) + 5} reduction chunks" in plan
    assert ("state" in plan) == state, plan
    v0 = (torch.rand((B, C_out, H, W), generator=torch.Generator().manual_seed(3)) * 0.6) if state else None
    v_th = 1.0 if neuron == "lif" else 0.5
    rep, _, r, v_fin = run_case(dev, case, neuron=neuron, v_th=v_th, v0=v0, traces=False, tail=True)
    assert rep.ok, str(rep)
    if state:
        assert torch.allclose(v_fin, r.v_final, rtol=1e-3, atol=1e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("slots", [1, 3, 7])
def test_tail_walks_many_tiles(dev, env, slots):
    """Few resident workgroups walking many tiles: the paired chunk's operand lookahead into the
    next tile's first full chunk, and tiles that start with the paired chunk (C_in = 64)."""
    env("SENGINE_AMD_PS_SLOTS", slots * 2)
    for C_in in (128, 64):
        case = _tail_case(470 + slots + C_in, 3, C_in, 128, 20, 18)
        rep, _, _, _ = run_case(dev, case, traces=False, tail=True)
        assert rep.ok, (C_in, str(rep))


@pytest.mark.gpu
def test_tail_refuses(dev):
    """A nonzero weight in the padding channels is a violation; strided, fp16 and T != 4
    descriptors are refused with a reason."""
    case = _tail_case(490, 1, 128, 64, 8, 8)
    case.w[3, 100, 1, 1] = 0.5
    spec = ops.ConvSpec(T=4, B=1, C_in=128, H=8, W=8, C_out=64, KH=3, KW=3, stride=1, padding=1)
    with pytest.raises(ops.SEngineError, match="padding"):
        ops.compress_2_4(spec, case.w.to(dev), tail=True)
    for bad in (dataclasses.replace(spec, stride=2), dataclasses.replace(spec, in_enc=ops.ENC_F16),
                dataclasses.replace(spec, T=2)):
        with pytest.raises(ops.SEngineError, match="tail"):
            ops.fused_plan(bad, tail=True)
