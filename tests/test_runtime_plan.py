"""CPU tests of the runtime's liveness-based buffer planner (sparsesnn_amd/runtime.py)."""
from sparsesnn_amd.runtime import plan_buffers


def _check_no_overlap(schedule, produces, consumes, aliases, plan):
    def find(t):
        while t in aliases:
            t = aliases[t]
        return t
    live = {}
    for i, nid in enumerate(schedule):
        for t in produces[nid]:
            live.setdefault(find(t), [i, i])
        for t in consumes[nid]:
            live.setdefault(find(t), [-1, i])[1] = i
    items = [(plan[t], a, b) for t, (a, b) in live.items()]
    for k, (b1, s1, e1) in enumerate(items):
        for b2, s2, e2 in items[k + 1:]:
            if b1 == b2:
                assert e1 <= s2 or e2 <= s1 or (e1 == s2 or e2 == s1), (b1, s1, e1, s2, e2)


def test_chain_reuses_two_buffers_per_size():
    schedule = [0, 1, 2, 3, 4]
    produces = {i: [f"t{i + 1}"] for i in schedule}
    consumes = {i: [f"t{i}"] for i in schedule}
    sizes = {f"t{i}": ("bits", 100) for i in range(6)}
    plan = plan_buffers(schedule, produces, consumes, {}, sizes, {"t0", "t5"})
    assert plan["t0"] != plan["t5"]
    assert len({plan[t] for t in sizes}) <= 4  # input, output and two ping-pong buffers
    for i in schedule:  # a node never writes the buffer it reads
        assert plan[f"t{i}"] != plan[f"t{i + 1}"]
    _check_no_overlap(schedule, produces, consumes, {}, plan)


def test_views_share_the_source_buffer_and_extend_its_life():
    schedule = [0, 1, 2, 3]
    produces = {0: ["a"], 1: ["a_view"], 2: ["b"], 3: ["c"]}
    consumes = {0: ["x"], 1: ["a"], 2: ["x"], 3: ["a_view"]}
    aliases = {"a_view": "a"}
    sizes = {t: ("bits", 10) for t in ("x", "a", "a_view", "b", "c")}
    plan = plan_buffers(schedule, produces, consumes, aliases, sizes, {"x", "c"})
    assert plan["a_view"] == plan["a"]
    assert plan["b"] != plan["a"]  # a is still live (read by node 3 through its view)
    assert plan["x"] != plan["c"]


def test_sizes_are_not_mixed():
    schedule = [0, 1, 2]
    produces = {0: ["a"], 1: ["b"], 2: ["c"]}
    consumes = {0: ["x"], 1: ["a"], 2: ["b"]}
    sizes = {"x": ("bits", 8), "a": ("f32", 64), "b": ("bits", 8), "c": ("bits", 8)}
    plan = plan_buffers(schedule, produces, consumes, {}, sizes, {"x", "c"})
    assert plan["a"] not in (plan["b"], plan["c"], plan["x"])


def test_engine_buffer_plan_reuses_sew_activations():
    """The generic engine's plan for SEW-ResNet-18 (analysis only, no GPU): launches read and
    write root tensors, buffers are reused across blocks, and no launch writes a buffer it
    reads."""
    from oracle import sew_resnet as sr
    from sparsesnn_amd import frontend, passes
    from sparsesnn_amd.runtime import CUDAGraphEngine
    ir = frontend.sew_resnet_ir(sr.make_params(1, fp16_weights=True), T=4, batch=2)
    passes.optimize_ir(ir)
    eng = CUDAGraphEngine()
    launches, aliases, shapes = eng._analyse(ir, ir.topo_order)
    launches = eng._order(launches, aliases, ir.topo_order)
    root = lambda t: CUDAGraphEngine._root(t, aliases)  # noqa: E731
    produces = {l.nid: [root(l.output)] for l in launches}
    consumes = {l.nid: [root(t) for t in l.inputs] for l in launches}
    sizes = {t: ("bits", 1) for ts in list(produces.values()) + list(consumes.values()) for t in ts}
    graph_in = {t for ts in consumes.values() for t in ts} - {t for ts in produces.values() for t in ts}
    plan = plan_buffers([l.nid for l in launches], produces, consumes, {}, sizes, graph_in | {"logits"})
    assert len(set(plan.values())) < len(sizes) // 2
    for l in launches:
        assert plan[root(l.output)] not in {plan[root(t)] for t in l.inputs}, ir.nodes[l.nid].name
    _check_no_overlap([l.nid for l in launches], produces, consumes, {}, plan)
