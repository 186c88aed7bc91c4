"""hipGraph inference engine over an optimized EngineIR.

Keeps the interface of the reference's CUDA-Graph runtime (sengine/cuda_graph_runtime.py:28-198:
CUDAGraphEngine.build(ir, kernels, schedule, T, batch_size, precision), capture_graph(),
__call__(x), reset_state(), benchmark()) so its callers drive this build unchanged, and the
reference's buffer planning idea (build/buffer_planner.py: activation buffers reused once a
tensor's last consumer has run).  Differences, MI355X-first:

  * spike tensors between nodes are packed bits (1/16 of the reference's fp16 bytes), and
    integer activations (SEW sums) bit planes; a spike-input graph packs its input once and
    unpacks its output once, both inside the captured graph;
  * fused nodes run with V0 = 0 and no membrane tensor: the reference zeroes every
    membrane before each replay (cuda_graph_runtime.py:158-159), which is the same thing;
    keep_membranes=True keeps per-node membranes instead (carried across calls until
    reset_state());
  * everything the schedule touches is allocated in build(): capture and replay allocate
    nothing.

Launches (one per non-absorbed node; the node kinds of cuda_graph_runtime.py:552-880 that
this path needs):
  * FusedSparseConvBNLIF (and the reference's TileLangFused* names), neuron absorbed, with
    the SEW 'ADD' absorbed into its epilogue when the passes recorded a residual_input; two
    fused convs reading the same input with no residual run as one paired launch;
  * FusedSparseConvBNLIF with a real-valued shortcut_input (MS-ResNet's membrane shortcut):
    the conv + BN + shortcut add + next neuron in one launch, writing the next neuron's spikes
    and the fp32 sum (real_output, the next block's real-valued input);
  * TileLangConvBN / TileLangConv1x1BN (dense fallback, fp32 out) + CUDAVec4LIF / CUDAVec4IF;
    TileLangConv1x1BN with real_input: the fp32 1x1 conv + BN of a real-valued tensor;
  * TileLangStemConvBN: the dense image stem with its repeat, neuron and max-pool absorbed
    (and its fp32 output kept, once per image, when the passes recorded a real_output);
  * FusedSparseConvBNLIF anchoring merged siblings (merged_nids: Spikformer's q, k, v): one
    launch over the concatenated weights, its spike bits split into one plane per conv -- the
    planes of one buffer, each conv's spike tensor a view of its plane;
  * FusedSpikformerAttn: the SSA core on spike bits (K^T V, then Q (K^T V) and the attention
    LIF: two kernels), its K^T V workspace allocated in build();
  * CuDNNPool: spike max-pool; CuBLASGemm: the head (pool + mean over T + Linear absorbed);
  * ZeroCost: views.  An unabsorbed Add / Tile / TemporalMean / GlobalAvgPool raises.
Spike tensors live as bits, real-valued tensors as fp32 NHWC, integer activations (residual
sums) as bit planes or, when the passes chose an fp16 stream (annotate_planes int_stream
'f16'), as fp16 integers NHWC.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from . import ops
from .compiler import (ATTENTION_VARIANTS, DENSE_VARIANTS, FUSED_VARIANTS, HEAD_VARIANTS, NEURON_VARIANTS,
                       POOL_VARIANTS, STEM_VARIANTS, _kname)
from .ops import ENC_BITS, ENC_F16, SEngineError


def plan_buffers(schedule: list, produces: dict, consumes: dict, aliases: dict, sizes: dict, keep: set) -> dict:
    """Liveness-based buffer assignment.

    schedule: node ids in execution order; produces[nid] / consumes[nid]: tensor names;
    aliases[name] = source name for views (same buffer); sizes[name] = a hashable buffer
    class (dtype, numel); keep: tensors that must never be overwritten (graph input and
    output).  Returns {tensor name: buffer index}; tensors of one buffer never overlap
    in time."""
    root = {}

    def find(t):
        while t in aliases:
            t = aliases[t]
        return t

    last_use = {}
    for i, nid in enumerate(schedule):
        for t in consumes.get(nid, []):
            last_use[find(t)] = i
        for t in produces.get(nid, []):
            last_use.setdefault(find(t), i)
    free: dict = {}
    assign: dict = {}
    n_buf = 0
    produced = {find(t) for ts in produces.values() for t in ts}
    for t in sorted(keep):  # kept tensors nobody produces (the graph input) exist from the start
        r = find(t)
        if r not in produced and r not in assign:
            assign[r] = n_buf
            n_buf += 1
    for i, nid in enumerate(schedule):
        for t in produces.get(nid, []):
            r = find(t)
            if r in assign or r != t:
                continue
            cls = sizes[r]
            pool = free.get(cls, [])
            if pool and r not in keep:
                assign[r] = pool.pop()
            else:
                assign[r] = n_buf
                n_buf += 1
        # release tensors whose last consumer is this node
        for t in {find(x) for x in consumes.get(nid, [])}:
            if last_use.get(t) == i and t in assign and t not in keep:
                free.setdefault(sizes[t], []).append(assign[t])
    for t in list(sizes):
        root[t] = assign.get(find(t))
    return root


_VIEW_OPS = {"Reshape", "Transpose", "Identity", "Flatten"}


class _Launch:
    """One kernel launch of the schedule: the anchor node, what it reads and writes."""

    def __init__(self, nid: int, kind: str, inputs: list, output: str, real_output: Optional[str] = None,
                 subs: Optional[list] = None):
        self.nid, self.kind, self.inputs, self.output = nid, kind, inputs, output
        self.real_output = real_output        # a second, fp32 output (membrane-shortcut sums, a kept stem output)
        self.subs = subs or []                # split launch: the tensors held by the planes of `output`
        self.pair_with: Optional[int] = None  # nid of a fused conv launched together with this one
        self.skip = False                     # launched as the second half of a pair

    @property
    def outputs(self) -> list:
        return [self.output] + ([self.real_output] if self.real_output else [])


class CUDAGraphEngine:
    """Static-shape inference over an EngineIR with every launch captured in one hipGraph."""

    def __init__(self):
        self.ir = None
        self.schedule: list = []
        self.launches: list = []
        self.kernels: dict = {}
        self.T, self.B, self.TB = 4, 1, 4
        self.graph: Optional[torch.cuda.CUDAGraph] = None
        self.buffers: list = []
        self.tensors: dict = {}
        self.weights: dict = {}
        self.bn: dict = {}
        self.membranes: dict = {}
        self.planes: dict = {}
        self._graph_input: Optional[torch.Tensor] = None
        self._graph_output: Optional[torch.Tensor] = None
        self.image_input = False
        self.logits_output = False
        self.enc: dict = {}
        self.sub: dict = {}
        self.attn_ws: Optional[torch.Tensor] = None
        self.head_ws: Optional[torch.Tensor] = None

    # ------------------------------------------------------------------ graph analysis
    def _launch_of(self, node) -> Optional[_Launch]:
        name = _kname(node)
        ea = node.extra_attrs
        if name in FUSED_VARIANTS and "merged_nids" in ea:
            return _Launch(node.id, "split", [node.input_names[0]], node.name + ".split", subs=list(ea["merged_outputs"]))
        if name in ATTENTION_VARIANTS:
            return _Launch(node.id, "attn", list(node.input_names), node.output_names[0])
        if name in FUSED_VARIANTS and "shortcut_input" in ea:
            return _Launch(node.id, "fused_sc", [node.input_names[0], ea["shortcut_input"]], ea["fused_output"],
                           ea["real_output"])
        if name in FUSED_VARIANTS:
            ins = [node.input_names[0]] + ([ea["residual_input"]] if "residual_input" in ea else [])
            return _Launch(node.id, "fused", ins, ea.get("fused_output", node.output_names[0]))
        if name in DENSE_VARIANTS and ea.get("real_input"):
            return _Launch(node.id, "real_conv", [node.input_names[0]], node.output_names[0])
        if name in DENSE_VARIANTS:
            return _Launch(node.id, "dense", [node.input_names[0]], node.output_names[0])
        if name in NEURON_VARIANTS:
            return _Launch(node.id, "neuron", [node.input_names[0]], node.output_names[0])
        if name in STEM_VARIANTS:
            return _Launch(node.id, "stem", [node.input_names[0]], ea["fused_output"], ea.get("real_output"))
        if name in HEAD_VARIANTS:
            return _Launch(node.id, "head", [ea["head_input"]], node.output_names[0])
        if name in POOL_VARIANTS:
            if node.op_type.name != "MaxPool":
                raise SEngineError(f"node {node.name}: only max-pool is served as a standalone pool")
            return _Launch(node.id, "pool", [node.input_names[0]], node.output_names[0])
        if name == "ZeroCost":
            return None
        raise SEngineError(f"node {node.name}: kernel {name} is not served by this build")

    def _analyse(self, ir, order):
        self.sub = {}
        absorbed = set()
        for node in ir.nodes.values():
            absorbed.update(node.extra_attrs.get("absorbed_nids", []))
        launches, aliases, shapes = [], {}, {}
        written = set()
        for nid in order:
            node = ir.nodes[nid]
            for i, t in enumerate(node.input_names):
                if i < len(node.input_shapes):
                    shapes.setdefault(t, tuple(node.input_shapes[i]))
            for i, t in enumerate(node.output_names):
                shapes[t] = tuple(node.output_shapes[i])
            ln = self._launch_of(node)
            if ln is not None:
                launches.append(ln)
                written.update(ln.outputs + ln.subs)
                if ln.kind == "split":  # the merged buffer: one plane of split_channels per conv
                    ea = node.extra_attrs
                    split = int(ea["split_channels"])
                    nplanes = -(-int(ea["merged_out_channels"]) // split)
                    N, _, H, W = node.output_shapes[0]
                    shapes[ln.output] = (N, nplanes * split, H, W)
                    for j, t in enumerate(ln.subs):
                        aliases[t] = ln.output
                        self.sub[t] = (j, nplanes)
        for nid in order:  # views (and absorbed single-input nodes) alias their input
            node = ir.nodes[nid]
            if _kname(node) != "ZeroCost":
                continue
            if nid not in absorbed and node.op_type.name not in _VIEW_OPS:
                raise SEngineError(f"node {node.name}: {node.op_type.name} is not absorbed into a fused launch and "
                                   "has no standalone kernel here")
            if len(node.input_names) == 1 and node.output_names[0] not in written:
                aliases[node.output_names[0]] = node.input_names[0]
        return launches, aliases, shapes

    @staticmethod
    def _root(t, aliases):
        while t in aliases:
            t = aliases[t]
        return t

    def _order(self, launches, aliases, schedule):
        """Launches in a dependency order (Kahn over what each reads and writes); the given
        schedule (or the IR's topological order) breaks ties."""
        prod = {self._root(o, aliases): l for l in launches for o in l.outputs}
        rank = {nid: i for i, nid in enumerate(schedule)}
        deps = {l.nid: {prod[self._root(t, aliases)].nid for t in l.inputs if self._root(t, aliases) in prod}
                for l in launches}
        by_id = {l.nid: l for l in launches}
        done, out = set(), []
        while len(out) < len(launches):
            ready = [l for l in launches if l.nid not in done and deps[l.nid] <= done]
            if not ready:
                raise SEngineError("launch dependencies form a cycle")
            nxt = min(ready, key=lambda l: rank.get(l.nid, 0))
            out.append(by_id[nxt.nid])
            done.add(nxt.nid)
        return out

    # ------------------------------------------------------------------ build
    def build(self, ir, kernels: dict, schedule: Optional[list] = None, T: Optional[int] = None, batch_size: int = 1,
              precision: str = "fp16", keep_membranes: bool = False, device="cuda", pair_launches: bool = True):
        self.ir = ir
        self.kernels = kernels
        self.schedule = list(schedule) if schedule is not None else list(ir.topo_order)
        self.T = int(T if T is not None else ir.T)
        self.B = int(batch_size)
        self.TB = self.T * self.B
        self.precision = precision
        self.keep_membranes = keep_membranes
        self.dev = torch.device(device)

        launches, aliases, shapes = self._analyse(ir, self.schedule)
        launches = self._order(launches, aliases, self.schedule)
        root = lambda t: self._root(t, aliases)  # noqa: E731
        produced = {root(o) for l in launches for o in l.outputs}
        inputs = {root(t) for l in launches for t in l.inputs if root(t) not in produced}
        if len(inputs) != 1:
            raise SEngineError(f"expected one graph input tensor, found {sorted(inputs)}")
        self.input_name = inputs.pop()
        consumed = {root(t) for l in launches for t in l.inputs}
        outs = [l.output for l in launches if root(l.output) not in consumed]
        if len(outs) != 1:
            raise SEngineError(f"expected one graph output tensor, found {sorted(outs)}")
        self.output_name = outs[0]
        first = [l for l in launches if self.input_name in {root(t) for t in l.inputs}]
        self.image_input = any(l.kind == "stem" for l in first)
        if self.image_input and len(first) != 1:
            raise SEngineError("the image input must feed the stem only")
        self.logits_output = launches[-1].kind == "head" and launches[-1].output == self.output_name

        # activation ranges: bit planes per tensor; out_planes 0 = an fp16 integer stream
        self.planes, self.enc = {}, {}
        for l in launches:
            node = ir.nodes[l.nid]
            p = int(node.extra_attrs.get("out_planes", 1)) if l.kind == "fused" else 1
            self.planes[root(l.output)] = max(p, 1)
            self.enc[root(l.output)] = "f16" if p == 0 else "bits"
        self.planes.setdefault(self.input_name, 1)
        if keep_membranes and any(l.kind in ("split", "attn") for l in launches):
            raise SEngineError("keep_membranes is not served for merged sibling convs or attention cores")

        # pair two fused convs on the same input (a block's conv1 and downsample): one launch
        if pair_launches and not keep_membranes:
            for i, a in enumerate(launches):
                if a.kind != "fused" or a.skip or a.pair_with is not None or len(a.inputs) != 1 or \
                        self.enc.get(root(a.inputs[0]), "bits") != "bits" or self.enc[root(a.output)] != "bits" or \
                        getattr(self.kernels.get(a.nid), "tail", False):
                    continue
                for b in launches[i + 1:]:
                    if b.kind == "fused" and not b.skip and b.pair_with is None and len(b.inputs) == 1 and \
                            root(b.inputs[0]) == root(a.inputs[0]) and self.enc[root(b.output)] == "bits" and \
                            not getattr(self.kernels.get(b.nid), "tail", False):
                        a.pair_with, b.skip = b.nid, True
                        break
            # the partner is written by its pair's launch: schedule it right after, so buffer
            # liveness (which follows schedule positions) is exact
            ordered = []
            partner = {l.pair_with: l for l in launches if l.pair_with is not None}
            for l in launches:
                if l.skip:
                    continue
                ordered.append(l)
                if l.pair_with is not None:
                    ordered.append(next(m for m in launches if m.nid == l.pair_with))
            assert len(ordered) == len(launches) and len(partner) == sum(l.skip for l in launches)
            launches = ordered
        self.launches = launches

        # buffers: spike bits (x planes), fp32 dense / real-valued outputs, logits; graph input and
        # output kept
        self.real = {root(l.real_output) for l in launches if l.real_output} | \
                    {root(l.output) for l in launches if l.kind == "real_conv"}
        # real tensors that hold one timestep (a stem's output, stored once per image)
        self.real_one_t = {root(l.real_output) for l in launches if l.kind == "stem" and l.real_output}

        def cls(t):
            r = root(t)
            shp = shapes[r]
            kind = next((l.kind for l in launches if root(l.output) == r), None)
            n = int(np.prod(shp))
            if kind == "dense" or kind == "head" or r in self.real:
                return ("f32", n)
            if r == self.input_name and self.image_input:
                return ("f32", n)
            if self.enc.get(r) == "f16":
                return ("f16", n)
            N, C = shp[0], shp[1]
            if (C * self.planes.get(r, 1)) % 32:
                raise SEngineError(f"tensor {t}: {C} channels is not a multiple of 32 (spike bits)")
            return ("bits", n * self.planes.get(r, 1) // 32)

        produces = {l.nid: [root(o) for o in l.outputs] for l in launches}
        consumes = {l.nid: [root(t) for t in l.inputs] for l in launches}
        live = {root(t) for l in launches for t in l.inputs + l.outputs}
        sizes = {t: cls(t) for t in live}
        plan = plan_buffers([l.nid for l in launches], produces, consumes, {}, sizes,
                            {self.input_name, root(self.output_name)})
        n_buf = 1 + max(b for b in plan.values() if b is not None)
        bufcls = {plan[t]: sizes[t] for t in sizes}
        dtypes = {"f32": torch.float32, "bits": torch.int32, "f16": torch.float16}
        self.buffers = [torch.empty(n, dtype=dtypes[k], device=self.dev)
                        for k, n in (bufcls[i] for i in range(n_buf))]
        self.tensors = {}
        for t in live:
            k, n = sizes[t]
            self.tensors[t] = self.buffers[plan[t]][:n]
        self._shapes = shapes
        self._root_fn = root

        if self.image_input:
            B, C, H, W = shapes[self.input_name]
            self._graph_input = self.tensors[self.input_name].view(B, C, H, W)
        else:
            Ni, Ci, Hi, Wi = shapes[self.input_name]
            self._graph_input = torch.zeros(Ni, Hi, Wi, Ci, dtype=torch.float16, device=self.dev)
        if self.logits_output:
            self._graph_output = self.tensors[root(self.output_name)].view(*shapes[self.output_name])
        else:
            No, Co, Ho, Wo = shapes[self.output_name]
            self._graph_output = torch.empty(No, Ho, Wo, Co, dtype=torch.float16, device=self.dev)

        # weights, BN vectors, membranes
        for l in launches:
            node = ir.nodes[l.nid]
            if l.kind in ("fused", "fused_sc", "dense", "stem", "real_conv"):
                w = torch.from_numpy(np.ascontiguousarray(ir.weights[node.weight_info.name]))
                self.weights[l.nid] = self.kernels[l.nid].prepare_weight(w.to(self.dev), device=self.dev)
                self.bn[l.nid] = (torch.tensor(node.bn_scale, dtype=torch.float32, device=self.dev),
                                  torch.tensor(node.bn_bias, dtype=torch.float32, device=self.dev))
                if keep_membranes and l.kind in ("fused", "fused_sc"):
                    N, C, H, W = node.output_shapes[0]
                    self.membranes[l.nid] = torch.zeros(N // self.T * H * W, C, device=self.dev)
            elif l.kind == "neuron" and keep_membranes:
                N, C, H, W = node.output_shapes[0]
                self.membranes[l.nid] = torch.zeros(N // self.T * H * W * C, device=self.dev)
            elif l.kind == "split":  # the concatenated weights and BN vectors of the merged convs
                ea = node.extra_attrs
                w = torch.from_numpy(np.ascontiguousarray(ir.weights[ea["merged_weight"]]))
                self.weights[l.nid] = self.kernels[l.nid].prepare_weight(w.to(self.dev), device=self.dev)
                sc, bi = ea["merged_bn"]
                self.bn[l.nid] = (torch.tensor(sc, dtype=torch.float32, device=self.dev),
                                  torch.tensor(bi, dtype=torch.float32, device=self.dev))
            elif l.kind == "head":
                self.weights[l.nid] = (
                    torch.from_numpy(np.ascontiguousarray(ir.weights[node.weight_info.name])).float().to(self.dev),
                    torch.from_numpy(np.ascontiguousarray(ir.weights[node.bias_info.name])).float().to(self.dev))
        # workspaces, shared by the launches that need one (they run one after another on one stream)
        n_kv = max([self.kernels[l.nid].kv_numel for l in launches if l.kind == "attn"], default=0)
        self.attn_ws = torch.empty(n_kv, dtype=torch.int32, device=self.dev) if n_kv else None
        n_hw = max([self.kernels[l.nid].workspace_numel for l in launches if l.kind == "head"], default=0)
        self.head_ws = torch.empty(n_hw, dtype=torch.int32, device=self.dev) if n_hw else None
        self.graph = None
        return self

    @property
    def n_launches(self) -> int:
        """Kernel launches per forward (pack / unpack of a spike-input graph included; an
        attention core is two, and so is a head whose sums are split over a workspace)."""
        n = sum(1 for l in self.launches if not l.skip)
        n += sum(1 for l in self.launches if l.kind == "attn")
        n += sum(1 for l in self.launches if l.kind == "head" and self.kernels[l.nid].workspace_numel)
        if not self.image_input:
            n += 1
        if not self.logits_output:
            n += 1
        return n

    def launch_names(self) -> list:
        """One label per kernel launch of a forward, in launch order (len == n_launches): the
        anchor node's name and launch kind; a pair names both convs, an attention core and a
        split-sum head give one label per kernel."""
        names = [] if self.image_input else ["pack_spikes"]
        for l in self.launches:
            if l.skip:
                continue
            name = self.ir.nodes[l.nid].name
            if l.kind == "split":
                name = " + ".join(self.ir.nodes[i].name for i in self.ir.nodes[l.nid].extra_attrs["merged_nids"])
            if l.pair_with is not None:
                name += " + " + self.ir.nodes[l.pair_with].name
            if l.kind == "attn":
                names += [f"{name} (attn: key-value sums)", f"{name} (attn: attend)"]
            elif l.kind == "head" and self.kernels[l.nid].workspace_numel:
                names += [f"{name} (head: partial sums)", f"{name} (head: classifier)"]
            else:
                names.append(f"{name} ({l.kind})")
        if not self.logits_output:
            names.append("unpack_spikes")
        return names

    # ------------------------------------------------------------------ execution
    def _bits(self, t):
        """An activation tensor as NHWC: int32 spike bits (N, H, W, C * planes / 32), or fp16
        (N, H, W, C) for an fp16 stream; a merged launch's per-conv tensor is its plane."""
        r = self._root_fn(t)
        N, C, H, W = self._shapes[r]
        if t in self.sub:
            j, nplanes = self.sub[t]
            return self.tensors[r].view(nplanes, N, H, W, C // nplanes // 32)[j]
        if self.enc.get(r) == "f16":
            return self.tensors[r].view(N, H, W, C)
        return self.tensors[r].view(N, H, W, C * self.planes.get(r, 1) // 32)

    def _enc_of(self, t) -> int:
        return ENC_F16 if self.enc.get(self._root_fn(t)) == "f16" else ENC_BITS

    def _run_fused(self, l):
        node = self.ir.nodes[l.nid]
        kern = self.kernels[l.nid]
        x, y = self._bits(l.inputs[0]), self._bits(l.output)
        sc, bi = self.bn[l.nid]
        sw = self.weights[l.nid]
        in_enc, out_enc = self._enc_of(l.inputs[0]), self._enc_of(l.output)
        spec = kern.spec_for(in_enc, out_enc)
        if len(l.inputs) == 2:  # SEW add absorbed; an fp16 residual / output is the fp16 stream
            ea = node.extra_attrs
            r = self._root_fn(l.inputs[1])
            res_planes = 0 if self.enc.get(r) == "f16" else int(self.planes.get(r, 1))
            ops.fused_sparse_conv_bn_lif_add(spec, x.view(-1), sw.values, sw.meta, sc, bi, self._bits(l.inputs[1]),
                                             res_planes, int(ea.get("out_planes", 1)),
                                             state=self.membranes.get(l.nid), out=y)
            return
        if l.pair_with is not None:
            o = next(m for m in self.launches if m.nid == l.pair_with)
            k2 = self.kernels[o.nid]
            sw2 = self.weights[o.nid]
            sc2, bi2 = self.bn[o.nid]
            ops.fused_sparse_conv_bn_lif_pair(spec, k2.spec_for(ENC_BITS, ENC_BITS), x.view(-1), sw.values, sw.meta,
                                              sc, bi, sw2.values, sw2.meta, sc2, bi2, out0=y, out1=self._bits(o.output))
            return
        mem = self.membranes.get(l.nid)
        args = (x, sw, mem, sc, bi) if mem is not None else (x, sw, sc, bi)
        kern(*args, out_enc=out_enc, out=y)

    def _run_split(self, l):
        kern = self.kernels[l.nid]
        sc, bi = self.bn[l.nid]
        sw = self.weights[l.nid]
        split = int(self.ir.nodes[l.nid].extra_attrs["split_channels"])
        r = self._root_fn(l.output)
        ops.fused_sparse_conv_bn_lif_split(kern.spec_for(self._enc_of(l.inputs[0]), ENC_BITS),
                                           self._bits(l.inputs[0]).view(-1), sw.values, sw.meta, sc, bi, split,
                                           out=self.tensors[r])

    def _real(self, t):
        """A real-valued tensor as fp32 NHWC (N, H, W, C); one-timestep tensors (a stem's kept
        output) as their first N / T rows."""
        r = self._root_fn(t)
        N, C, H, W = self._shapes[r]
        if r in self.real_one_t:
            N //= self.T
        return self.tensors[r][:N * H * W * C].view(N, H, W, C)

    def _run_fused_sc(self, l):
        kern = self.kernels[l.nid]
        sc, bi = self.bn[l.nid]
        sw = self.weights[l.nid]
        res = self._root_fn(l.inputs[1])
        if res in self.real_one_t:
            raise SEngineError(f"node {self.ir.nodes[l.nid].name}: an identity shortcut needs a T-step real input")
        ops.fused_sparse_conv_bn_add_neuron(kern.spec_for(ENC_BITS, ENC_BITS), self._bits(l.inputs[0]).view(-1),
                                            sw.values, sw.meta, sc, bi, residual=self._real(res),
                                            state=self.membranes.get(l.nid), real_out=self._real(l.real_output),
                                            out=self._bits(l.output))

    def _execute_schedule(self):
        if not self.image_input:  # first op of the graph
            ops.pack_spikes(self._graph_input, out=self._bits(self.input_name))
        for l in self.launches:
            if not l.skip:
                self._run_launch(l)
        if not self.logits_output:
            ops.unpack_spikes(self._bits(self.output_name), self._graph_output.shape[-1], out=self._graph_output)

    def _run_launch(self, l):
        """One launch of the schedule (the second half of a pair runs with its first)."""
        node = self.ir.nodes[l.nid]
        if l.kind == "fused":
            self._run_fused(l)
        elif l.kind == "fused_sc":
            self._run_fused_sc(l)
        elif l.kind == "split":
            self._run_split(l)
        elif l.kind == "attn":
            kern = self.kernels[l.nid]
            q, k, v = (self._bits(t) for t in l.inputs)
            kern(q, k, v, kv=self.attn_ws[:kern.kv_numel], out=self._bits(l.output))
        elif l.kind == "real_conv":
            sc, bi = self.bn[l.nid]
            x = self._root_fn(l.inputs[0])
            self.kernels[l.nid](self._real(x), self.weights[l.nid], sc, bi,
                                in_T=1 if x in self.real_one_t else self.T, out=self._real(l.output))
        elif l.kind == "dense":
            sc, bi = self.bn[l.nid]
            r = self._root_fn(l.output)
            N, C, H, W = self._shapes[r]
            self.kernels[l.nid](self._bits(l.inputs[0]), self.weights[l.nid], sc, bi,
                                out=self.tensors[r].view(N, H, W, C))
        elif l.kind == "neuron":  # standalone neuron on a dense conv's fp32 output
            p = node.neuron_params
            kind = "lif" if node.op_type.name == "LIF" else "if"
            v_reset = float(p.v_reset) if p.hard_reset else None
            ops.multistep_neuron(self.tensors[self._root_fn(l.inputs[0])], self.T, kind, float(p.tau),
                                 float(p.v_threshold), v_reset, state=self.membranes.get(l.nid), out_enc=ENC_BITS,
                                 out=self._bits(l.output).view(-1))
        elif l.kind == "stem":
            sc, bi = self.bn[l.nid]
            kern = self.kernels[l.nid]
            y = self._bits(l.output)
            if kern.pool is not None:
                kern(self._graph_input, self.weights[l.nid], sc, bi, pooled=y)
            else:
                kern(self._graph_input, self.weights[l.nid], sc, bi, spikes=y,
                     out=self._real(l.real_output) if l.real_output else None)
        elif l.kind == "pool":
            r = self._root_fn(l.inputs[0])
            N, C, H, W = self._shapes[r]
            if self.planes.get(r, 1) != 1:
                raise SEngineError(f"node {node.name}: max-pool of integer activations is not served")
            pp = node.pool_params or {}
            ops.maxpool_spikes(self._bits(l.inputs[0]), N, H, W, C, int(pp.get("kernel_size", 3)),
                               int(pp.get("stride", 2)), int(pp.get("padding", 1)), out=self._bits(l.output))
        elif l.kind == "head":
            fw, fb = self.weights[l.nid]
            kern = self.kernels[l.nid]
            ws = self.head_ws[:kern.workspace_numel] if kern.workspace_numel else None
            kern(self._bits(l.inputs[0]).view(-1), fw, fb, out=self._graph_output, workspace=ws)

    def capture_graph(self):
        """Warm up on a side stream, then capture the whole schedule into one hipGraph."""
        side = torch.cuda.Stream(self.dev)
        side.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(side):
            self._execute_schedule()
        torch.cuda.current_stream(self.dev).wait_stream(side)
        torch.cuda.synchronize(self.dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._execute_schedule()
        self.graph = g
        return g

    def _load_input(self, x: torch.Tensor):
        if self.image_input:
            if tuple(x.shape) != tuple(self._graph_input.shape):
                raise SEngineError(f"input shape {tuple(x.shape)}: expected images {tuple(self._graph_input.shape)}")
            self._graph_input.copy_(x)
            return
        TB, H, W, C = self._graph_input.shape
        if tuple(x.shape) != (TB, H, W, C):  # NCHW, per image (repeated over T) or per (t, b)
            if x.ndim != 4 or tuple(x.shape[1:]) != (C, H, W) or x.shape[0] not in (self.B, TB):
                raise SEngineError(f"input shape {tuple(x.shape)}: expected NHWC {(TB, H, W, C)} or NCHW "
                                   f"({self.B} or {TB}, {C}, {H}, {W})")
            if x.shape[0] != TB:
                x = x.repeat(self.T, 1, 1, 1)
            x = x.permute(0, 2, 3, 1)
        self._graph_input.copy_(x)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        """Spike-input graphs: x spikes (B, C, H, W) (repeated over T, as the reference's
        static-image input) or (T*B, C, H, W) NCHW, or (T*B, H, W, C) NHWC; returns fp16 NHWC
        spikes (T*B, OH, OW, C).  Image-input graphs (a stem first): x (B, C, H, W) fp32
        pixels; returns the head's logits (B, classes) fp32."""
        self._load_input(x)
        if self.graph is not None:
            self.graph.replay()
        else:
            self._execute_schedule()
        return self._graph_output.clone()

    def reset_state(self):
        """Zero the kept membranes (no-op without keep_membranes: every call starts at V0 = 0)."""
        for m in self.membranes.values():
            m.zero_()

    def benchmark(self, warmup: int = 200, n_iters: int = 1000) -> float:
        """Mean latency in ms of one forward (graph replay if captured), HIP events."""
        run = self.graph.replay if self.graph is not None else self._execute_schedule
        for _ in range(warmup):
            run()
        torch.cuda.synchronize(self.dev)
        s = torch.cuda.current_stream(self.dev)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(s)
        for _ in range(n_iters):
            run()
        b.record(s)
        torch.cuda.synchronize(self.dev)
        return a.elapsed_time(b) / n_iters

    def spike_density(self) -> dict:
        """Activity of every spike tensor of the last forward's input: fraction of set bits per
        activation (for integer activations, of nonzero values).  The forward is run again
        eagerly, launch by launch, and each tensor measured right after its launch wrote it (the
        buffer planner recycles a tensor's memory once its readers have run); kept membranes advance
        as in a forward.  Off the timed path."""
        lut = torch.tensor([bin(i).count("1") for i in range(256)], dtype=torch.int64, device=self.dev)
        out = {}
        if not self.image_input:
            ops.pack_spikes(self._graph_input, out=self._bits(self.input_name))
        for l in self.launches:
            if l.skip:
                continue
            self._run_launch(l)
            done = [l] + ([m for m in self.launches if m.nid == l.pair_with] if l.pair_with is not None else [])
            for m in done:
                if m.kind not in ("dense", "head", "real_conv"):
                    self._density(m, lut, out)
        return out

    def _density(self, l, lut, out):
        for t in (l.subs or [l.output]):
            r = self._root_fn(t)
            v = self._bits(t)
            name = self.ir.nodes[l.nid].name + (f"[{t}]" if l.subs else "")
            if self.enc.get(r) == "f16":
                out[name] = float((v != 0).sum()) / v.numel()
                continue
            N, C, H, W = self._shapes[r]
            P = self.planes.get(r, 1)
            if t in self.sub:
                C //= self.sub[t][1]
            words = v.reshape(N * H * W, P, C // 32)
            nz = words[:, 0]
            for p in range(1, P):
                nz = nz | words[:, p]
            cnt = int(lut[nz.contiguous().view(torch.uint8).long()].sum())
            out[name] = cnt / float(N * H * W * C)


HipGraphEngine = CUDAGraphEngine
