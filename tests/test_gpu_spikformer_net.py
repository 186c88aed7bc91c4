"""GPU parity of Spikformer as a whole network: the SPS stages, every block
teacher-forced on the oracle's own token stream, the whole forward from one hipGraph replay
against the oracle's logits, and the config-4 shape (224x224, embed 384, 8 heads, 8 blocks):
at the benchmark's batch of 32 every SPS stage and all 8 blocks are checked on sampled images
(images are independent through the network, so each launch's rows for an image are compared
with the oracle run on that image's inputs), and on one and four images."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import packing as pk
from oracle import reference_path as ref
from oracle import spikformer as sf
from sparsesnn_amd.spikformer import SpikformerEngine
from tests.parity import compare

pytestmark = pytest.mark.gpu


def _img_bits(bits, T, B, C, H, W, c_real=None):
    """(T*B, H, W, C/32) bits -> (T, B, C, H, W) float; keep the first c_real channels."""
    a = pk.unpack_bits(bits.cpu().numpy().view(np.uint32).reshape(-1, C // 32), C)
    a = np.ascontiguousarray(a.reshape(T, B, H, W, C).transpose(0, 1, 4, 2, 3))
    return torch.from_numpy(a[:, :, :c_real] if c_real else a)


def _tok_bits(bits, T, B, N, C):
    """(T*B, N, C/32) bits -> (T, B, N, C) float."""
    a = pk.unpack_bits(bits.cpu().numpy().view(np.uint32).reshape(-1, C // 32), C)
    return torch.from_numpy(a.reshape(T, B, N, C))


def _tok_planes(bits, planes, T, B, N, C):
    """(T*B, N, planes*C/32) -> integer (T, B, N, C) float."""
    a = pk.planes_to_seq(bits.cpu().numpy().view(np.uint32).reshape(-1, planes * C // 32), planes, T, B, C, N, 1)
    return torch.from_numpy(a[..., 0].transpose(0, 1, 3, 2).copy())


def _planes_of(x, planes, dev):
    """integer tokens (T, B, N, C) -> device bit planes (T*B, N, planes*C/32)."""
    T, B, N, C = x.shape
    seq = x.permute(0, 1, 3, 2).unsqueeze(-1).numpy()  # (T, B, C, N, 1)
    return torch.from_numpy(pk.seq_to_planes(seq, planes).view(np.int32)).to(dev)


def _tok_stream(eng, buf, planes, T, B, N, C):
    """The engine's integer token stream -> (T, B, N, C) float (fp16 stream or bit planes)."""
    if eng.stream == "f16":
        return buf.float().cpu().view(T, B, N, C)
    return _tok_planes(buf, planes, T, B, N, C)


def _stream_of(eng, x, planes, dev):
    """integer tokens (T, B, N, C) -> the engine's stream representation on the device."""
    if eng.stream == "f16":
        T, B, N, C = x.shape
        return x.reshape(T * B, N, C).half().contiguous().to(dev)
    return _planes_of(x, planes, dev)


def _rows(t, T, B, sel):
    """Rows (T*B, ...) of a device tensor -> the rows of images `sel` (T*len(sel), ...)."""
    if sel is None:
        return t
    v = t.reshape(T, B, *t.shape[1:])[:, list(sel)]
    return v.reshape(T * len(sel), *t.shape[1:])


def _stage(p, name, x_seq):
    bn = sf.bn_of(p, f"patch_embed.{name.replace('conv', 'bn')}")
    return ref.fused_layer(x_seq, p[f"patch_embed.{name}.weight"], bn, 1, 1, 1, "lif", 2.0, 1.0, 0.0)


def _pool(x):
    T = x.shape[0]
    y = F.max_pool2d(x.flatten(0, 1), 3, 2, 1)
    return y.view(T, -1, *y.shape[1:])


def _check_sps(eng, p, x_img, T, B, embed, sel=None):
    """Each SPS stage of the engine against the oracle stage run on the engine's own input (of
    images `sel` only, when given)."""
    H, W = eng.stem_spec.H, eng.stem_spec.W
    c8, c4, c2 = embed // 8, embed // 4, embed // 2
    P8, P4 = eng.stem_spec.C_out, eng.c1.spec.C_out
    if sel is not None:
        x_img = x_img[list(sel)]
    Bs = B if sel is None else len(sel)
    r0 = _stage(p, "proj_conv", x_img.float().unsqueeze(0).repeat(T, 1, 1, 1, 1))
    B = Bs
    s0 = _img_bits(_rows(eng.s0, T, eng.B, sel), T, B, P8, H, W)
    assert float(s0[:, :, c8:].abs().sum()) == 0  # padded channels never fire
    rep = compare(s0[:, :, :c8].numpy(), None, r0.spikes.numpy(), r0.h.numpy(), 1.0)
    assert rep.ok, f"proj_conv {rep}"
    r1 = _stage(p, "proj_conv1", s0[:, :, :c8])
    s1 = _img_bits(_rows(eng.s1, T, eng.B, sel), T, B, P4, H, W)
    assert float(s1[:, :, c4:].abs().sum()) == 0
    rep = compare(s1[:, :, :c4].numpy(), None, r1.spikes.numpy(), r1.h.numpy(), 1.0)
    assert rep.ok, f"proj_conv1 {rep}"
    r2 = _stage(p, "proj_conv2", s1[:, :, :c4])
    s2 = _img_bits(_rows(eng.s2, T, eng.B, sel), T, B, c2, H, W)
    rep = compare(s2.numpy(), None, r2.spikes.numpy(), r2.h.numpy(), 1.0)
    assert rep.ok, f"proj_conv2 {rep}"
    p2 = _img_bits(_rows(eng.p2, T, eng.B, sel), T, B, c2, eng.H2, eng.W2)
    assert torch.equal(p2, _pool(s2))
    r3 = _stage(p, "proj_conv3", p2)
    s3 = _img_bits(_rows(eng.s3, T, eng.B, sel), T, B, embed, eng.H2, eng.W2)
    rep = compare(s3.numpy(), None, r3.spikes.numpy(), r3.h.numpy(), 1.0)
    assert rep.ok, f"proj_conv3 {rep}"
    p3 = _img_bits(_rows(eng.p3, T, eng.B, sel), T, B, embed, eng.H4, eng.W4)
    assert torch.equal(p3, _pool(s3))
    rr = _stage(p, "rpe_conv", p3)
    x0 = _tok_stream(eng, _rows(eng.x0, T, eng.B, sel), 2, T, B, eng.N, embed)
    srpe = x0 - p3.flatten(-2).transpose(-1, -2)
    assert set(np.unique(srpe.numpy())) <= {0.0, 1.0}
    rep = compare(srpe.transpose(-1, -2).reshape(rr.spikes.shape).numpy(), None, rr.spikes.numpy(), rr.h.numpy(),
                  1.0)
    assert rep.ok, f"rpe_conv {rep}"
    return [float(r.spikes.mean()) for r in (r0, r1, r2, r3, rr)]


def _check_block(dev, eng, p, i, x, T, B, heads, sel=None):
    """Block i on the token stream x (T, B, N, C): q/k/v and fc1 spikes under the parity rule
    on the engine's own inputs, SSA bit-exact on the engine's q/k/v, the two residual adds
    exact.  x given: the block is re-run on it (teacher forcing); x None: the block's buffers
    from the engine's last forward are checked against its own input stream, on images `sel`.
    Returns the mean attention spike rate."""
    blk = eng.blocks[i]
    pre = blk.name
    if x is not None:
        eng.run_block(i, x=_stream_of(eng, x, blk.planes_in, dev))
        torch.cuda.synchronize()
    else:
        xin, planes = eng.block_input(i)
        x = _tok_stream(eng, _rows(xin, T, B, sel), planes, T, len(sel), eng.N, eng.embed)
        B = len(sel)
    N, C = x.shape[2], x.shape[3]
    b = {k: _rows(v, T, eng.B, sel) if k != "qkv" else None for k, v in blk.bufs.items()}

    def lin(name, inp, got, v_th=1.0):
        s, h, _ = sf.linear_bn_lif(inp, p[f"{pre}.{name}_linear.weight"], p[f"{pre}.{name}_linear.bias"],
                                   sf.bn_of(p, f"{pre}.{name}_bn"), 2.0, v_th)
        rep = compare(got.numpy(), None, s.numpy(), h.numpy(), v_th)
        assert rep.ok, f"{pre}.{name} {rep}"
        return s

    q = _tok_bits(b["q"], T, B, N, C)
    k = _tok_bits(b["k"], T, B, N, C)
    v = _tok_bits(b["v"], T, B, N, C)
    for name, got in (("attn.q", q), ("attn.k", k), ("attn.v", v)):
        lin(name, x, got)
    a_ref = sf.ssa(q, k, v, heads)[0]
    a = _tok_bits(b["a"], T, B, N, C)
    assert torch.equal(a, a_ref), f"{pre} ssa"
    x1 = _tok_stream(eng, b["x1"], blk.planes_mid, T, B, N, C)
    sp = x1 - x
    assert set(np.unique(sp.numpy())) <= {0.0, 1.0}
    lin("attn.proj", a, sp)
    h = _tok_bits(b["h"], T, B, N, C * 4)
    lin("mlp.fc1", x1, h)
    x2 = _tok_stream(eng, b["x2"], blk.planes_out, T, B, N, C)
    s2 = x2 - x1
    assert set(np.unique(s2.numpy())) <= {0.0, 1.0}
    lin("mlp.fc2", h, s2)
    return float(a_ref.mean())


@pytest.fixture(scope="module")
def sf_case():
    p = sf.make_params(31, embed=128, depth=4, num_classes=10)
    x = torch.randn(2, 3, 32, 32, generator=torch.Generator().manual_seed(32))
    logits, xs = sf.forward(p, x, T=4, heads=2, depth=4, keep=True)
    return p, x, logits, xs


@pytest.mark.parametrize("stream,tail", [("f16", False), ("planes", False), ("f16", True)])
def test_engine_sps_and_blocks_teacher_forced(dev, env, sf_case, stream, tail):
    """SPS stages and blocks against the oracle; tail: proj_conv2 (32 channels padded to 64) on
    the opt-in paired-tail call."""
    p, x, _, xs = sf_case
    env("SENGINE_AMD_TAIL", int(tail))
    eng = SpikformerEngine(p, batch=2, T=4, embed=128, heads=2, depth=4, in_hw=(32, 32), device=dev, stream=stream)
    assert eng.c2.tail == tail
    eng.forward(x.to(dev))
    torch.cuda.synchronize()
    rates = _check_sps(eng, p, x, 4, 2, 128)
    assert all(0.005 < r < 0.9 for r in rates), rates
    for i in range(4):
        ra = _check_block(dev, eng, p, i, xs[i], 4, 2, 2)
        assert 0.005 < ra < 0.95


@pytest.mark.parametrize("stream", ["f16", "planes"])
def test_engine_end_to_end_graph(dev, sf_case, stream):
    p, x, logits, xs = sf_case
    eng = SpikformerEngine(p, batch=2, T=4, embed=128, heads=2, depth=4, in_hw=(32, 32), device=dev, stream=stream)
    eager = eng.forward(x.to(dev)).clone()
    eng.capture()
    for _ in range(3):
        y = eng.forward(x.to(dev))
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
    final = _tok_stream(eng, eng.blocks[-1].bufs["x2"], eng.final_planes, 4, 2, eng.N, 128)
    assert float((final != xs[-1]).float().mean()) <= 1e-3
    err = float((eager.cpu() - logits).abs().max())
    assert err < 5e-2, err
    # q/k/v in one launch; the fp16 stream's head sums in two launches
    assert eng.launches == 7 + 6 * 4 + (2 if stream == "f16" else 1)


@pytest.mark.parametrize("batch,nblocks,stream,tail", [(1, 1, "f16", False), (4, 2, "f16", False),
                                                       (1, 1, "planes", False), (1, 0, "f16", True)])
def test_engine_cfg4_shape(dev, env, batch, nblocks, stream, tail):
    """BASELINE config 4's shape: 3x224x224 pixels ~N(0,1), T=4, embed 384, 8 heads, MLP ratio
    4, 8 blocks (3,136 tokens), 1000 classes, on one image and on four; the SPS stages and
    the first `nblocks` blocks teacher-forced against the oracle, graph replays equal to the
    eager run.  tail: proj_conv2 (96 channels padded to 128) on the opt-in paired-tail call."""
    env("SENGINE_AMD_TAIL", int(tail))
    p = sf.make_params(41, embed=384, depth=8, num_classes=1000)
    x = torch.randn(batch, 3, 224, 224, generator=torch.Generator().manual_seed(42))
    eng = SpikformerEngine(p, batch=batch, T=4, embed=384, heads=8, depth=8, in_hw=(224, 224), device=dev,
                           stream=stream)
    assert eng.c2.tail == tail
    assert eng.N == 3136 and eng.final_planes == (5 if stream == "planes" else 0)
    eager = eng.forward(x.to(dev)).clone()
    eng.capture()
    y = eng.forward(x.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(y, eager)
    rates = _check_sps(eng, p, x, 4, batch, 384)
    assert all(0.005 < r < 0.9 for r in rates), rates
    xi = _tok_stream(eng, eng.x0, 2, 4, batch, eng.N, 384)  # the engine's own (parity-checked) SPS output
    for i in range(nblocks):
        _check_block(dev, eng, p, i, xi, 4, batch, 8)
        blk = eng.blocks[i]
        xi = _tok_stream(eng, blk.bufs["x2"], blk.planes_out, 4, batch, eng.N, 384)  # checked block output


def test_engine_cfg4_bench_batch(dev):
    """BASELINE config 4 at the benchmark's own shape and batch (B = 32, fp16 stream, 8 blocks):
    every launch the bench times runs here.  After one eager forward every SPS stage and all 8
    blocks are checked against the oracle on the engine's own inputs for images 0, 13 and 31
    (images are independent through SPS, the token Linears and the per-image attention), the
    fused-kernel instances are asserted to be the ones named for B = 32, and a graph replay
    reproduces the eager logits."""
    from sparsesnn_amd import ops
    B, sel = 32, (0, 13, 31)
    p = sf.make_params(43, embed=384, depth=8, num_classes=1000)
    x = torch.randn(B, 3, 224, 224, generator=torch.Generator().manual_seed(44))
    eng = SpikformerEngine(p, batch=B, T=4, embed=384, heads=8, depth=8, in_hw=(224, 224), device=dev)
    assert eng.N == 3136 and eng.stream == "f16"
    for f in [eng.c1, eng.c2, eng.c3, eng.rpe] + [l for blk in eng.blocks for l in (blk.qkv, blk.proj, blk.fc1,
                                                                                     blk.fc2)]:
        assert f.spec.B == B
        print(f"{f.spec.C_in}->{f.spec.C_out} {f.spec.H}x{f.spec.W} k{f.spec.KH}: {ops.fused_plan(f.spec)}",
              flush=True)
    eager = eng.forward(x.to(dev)).clone()
    torch.cuda.synchronize()
    rates = _check_sps(eng, p, x, 4, B, 384, sel=sel)
    print("SPS spike rates", [round(r, 4) for r in rates], flush=True)
    assert all(0.005 < r < 0.9 for r in rates), rates
    for i in range(8):
        ra = _check_block(dev, eng, p, i, None, 4, B, 8, sel=sel)
        print(f"block {i}: attention spike rate {ra:.4f}", flush=True)
    eng.capture()
    y = eng.forward(x.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(y, eager)
