"""GPU: Spikformer through the generic graph engine (frontend.spikformer_ir -> optimize_ir ->
compile_all -> CUDAGraphEngine), bit-identical to the hand-wired SpikformerEngine, whose SPS
stages and every block are checked against the oracle in tests/test_gpu_spikformer_net.py.
Both streams (fp16 integers and bit planes) on small images, and BASELINE config 4
(Spikformer-8-384, 8 heads, 3x224x224, T=4, batch 32) with graph replays.  Parameters: the
oracle's 'lively' draw (every layer spikes; the reference's own initialisation leaves the
blocks of these small models nearly silent, which would make the comparison vacuous)."""
import pytest
import torch

from oracle import spikformer as sf
from sparsesnn_amd import frontend, passes
from sparsesnn_amd.compiler import SparseKernelCompiler
from sparsesnn_amd.runtime import CUDAGraphEngine
from sparsesnn_amd.spikformer import SpikformerEngine

pytestmark = pytest.mark.gpu


def build_generic(p, B, heads, hw, dev, int_stream="f16"):
    ir = frontend.spikformer_ir(p, T=4, batch=B, in_hw=hw, heads=heads)
    passes.optimize_ir(ir, int_stream=int_stream)
    kernels = SparseKernelCompiler(ir, batch_size=B).compile_all()
    return CUDAGraphEngine().build(ir, kernels, T=4, batch_size=B, device=dev)


@pytest.mark.parametrize("stream,embed,heads,depth,B,hw,tail", [
    ("f16", 128, 2, 4, 2, (32, 32), False),
    ("planes", 128, 2, 4, 2, (32, 32), False),
    ("f16", 128, 2, 4, 2, (32, 32), True),
    ("f16", 256, 4, 2, 3, (64, 48), False),
    ("f16", 384, 8, 8, 32, (224, 224), False),
])
def test_generic_engine_runs_spikformer(dev, env, stream, embed, heads, depth, B, hw, tail):
    """tail: both engines run proj_conv2 (embed/4 channels padded to 64) on the opt-in
    paired-tail call."""
    print(f"stream {stream} embed {embed} heads {heads} depth {depth} B {B} {hw} tail {tail}", flush=True)
    env("SENGINE_AMD_TAIL", int(tail))
    p = sf.make_params(80 + depth, embed=embed, depth=depth, num_classes=1000 if hw[0] == 224 else 10)
    x = torch.randn((B, 3) + hw, generator=torch.Generator().manual_seed(81))
    eng = build_generic(p, B, heads, hw, dev, stream)
    ref_eng = SpikformerEngine(p, batch=B, T=4, embed=embed, heads=heads, depth=depth, in_hw=hw, device=dev,
                               stream=stream)
    assert any(getattr(k, "tail", False) for k in eng.kernels.values()) == tail == ref_eng.c2.tail
    assert eng.n_launches == ref_eng.launches, (eng.n_launches, ref_eng.launches)
    names = eng.launch_names()
    assert len(names) == eng.n_launches and any("(attn: attend)" in n for n in names), names
    want = ref_eng.forward(x.to(dev)).clone()
    eager = eng(x.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(eager, want), float((eager - want).abs().max())
    # not only the logits: the SPS output, the last block's q / k / v and attention spikes, each
    # checked right after its launch (the buffer planner recycles their memory later), and the
    # final stream
    last = ref_eng.blocks[-1]
    attn_last = [l for l in eng.launches if l.kind == "attn"][-1]
    eng._load_input(x.to(dev))
    for i, l in enumerate(eng.launches):
        eng._run_launch(l)
        if i == 6:
            assert eng.ir.nodes[l.nid].name == "patch_embed.rpe_conv"
            assert torch.equal(eng._bits(l.output).reshape(-1), ref_eng.x0.reshape(-1))
        if l is attn_last:
            assert torch.equal(eng._bits(l.output).reshape(-1), last.bufs["a"].reshape(-1))
            for j, n in enumerate("qkv"):
                assert torch.equal(eng._bits(l.inputs[j]).reshape(-1), last.bufs[n].reshape(-1)), n
    head = eng.launches[-1]
    assert head.kind == "head"
    assert torch.equal(eng._bits(head.inputs[0]).reshape(-1), last.bufs["x2"].reshape(-1))
    assert torch.equal(eng._graph_output, want)
    rates = eng.spike_density()
    print({k: round(v, 4) for k, v in rates.items() if "block.0" in k or "patch" in k}, flush=True)
    for name in ("block.0.attn.core", f"block.{depth - 1}.attn.core", "block.0.mlp.fc1_linear"):
        assert 0.005 < rates[name] < 0.95, (name, rates[name])
    eng.capture_graph()
    for i in range(3):
        y = eng(x.to(dev))
        torch.cuda.synchronize()
        assert torch.equal(y, want), f"replay {i}"
        _ = (torch.ones(1000, device=dev) * i).sum().item()
