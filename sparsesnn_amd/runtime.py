"""hipGraph inference engine over an optimized EngineIR.

Keeps the interface of the reference's CUDA-Graph runtime (sengine/cuda_graph_runtime.py:28-198:
CUDAGraphEngine.build(ir, kernels, schedule, T, batch_size, precision), capture_graph(),
__call__(x), reset_state(), benchmark()) so its callers drive this build unchanged, and the
reference's buffer planning idea (build/buffer_planner.py: activation buffers reused once a
tensor's last consumer has run).  Differences, MI355X-first:

  * spike tensors between nodes are packed bits (1/16 of the reference's fp16 bytes); the
    graph packs the input once and unpacks the output once, both inside the captured graph;
  * fused nodes run with V0 = 0 and no membrane tensor: the reference zeroes every
    membrane before each replay (cuda_graph_runtime.py:158-159), which is the same thing;
    keep_membranes=True keeps per-node membranes instead (carried across calls until
    reset_state());
  * everything the schedule touches is allocated in build(): capture and replay allocate
    nothing.

Node kinds served: FusedSparseConvBNLIF (and the reference's TileLangFused* names) with the
neuron absorbed, TileLangConvBN / TileLangConv1x1BN (dense fallback, fp32 out) followed by
a CUDAVec4LIF / CUDAVec4IF neuron node, and ZeroCost nodes (views).  Anything else raises.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from . import ops
from .compiler import DENSE_VARIANTS, FUSED_VARIANTS, NEURON_VARIANTS, _kname
from .ops import ENC_BITS, SEngineError


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


class CUDAGraphEngine:
    """Static-shape inference over an EngineIR with every launch captured in one hipGraph."""

    def __init__(self):
        self.ir = None
        self.schedule: list = []
        self.kernels: dict = {}
        self.T, self.B, self.TB = 4, 1, 4
        self.graph: Optional[torch.cuda.CUDAGraph] = None
        self.buffers: list = []
        self.tensors: dict = {}
        self.weights: dict = {}
        self.bn: dict = {}
        self.membranes: dict = {}
        self._graph_input: Optional[torch.Tensor] = None
        self._graph_output: Optional[torch.Tensor] = None

    # ------------------------------------------------------------------ build
    def build(self, ir, kernels: dict, schedule: Optional[list] = None, T: Optional[int] = None, batch_size: int = 1,
              precision: str = "fp16", keep_membranes: bool = False, device="cuda"):
        self.ir = ir
        self.kernels = kernels
        self.schedule = list(schedule) if schedule is not None else list(ir.topo_order)
        self.T = int(T if T is not None else ir.T)
        self.B = int(batch_size)
        self.TB = self.T * self.B
        self.precision = precision
        self.keep_membranes = keep_membranes
        self.dev = torch.device(device)

        produces, consumes, aliases, shapes = {}, {}, {}, {}
        for nid in self.schedule:
            node = ir.nodes[nid]
            name = _kname(node)
            consumes[nid] = list(node.input_names[:1])
            produces[nid] = list(node.output_names[:1])
            shapes[node.output_names[0]] = tuple(node.output_shapes[0])
            for i, t in enumerate(node.input_names[:1]):
                shapes.setdefault(t, tuple(node.input_shapes[i]))
            if name == "ZeroCost":
                aliases[node.output_names[0]] = node.input_names[0]
            elif name not in FUSED_VARIANTS | DENSE_VARIANTS | NEURON_VARIANTS:
                raise SEngineError(f"node {node.name}: kernel {name} is not served by this build")
        produced = {t for ts in produces.values() for t in ts}
        inputs = [t for ts in consumes.values() for t in ts if t not in produced]
        if len(set(inputs)) != 1:
            raise SEngineError(f"expected one graph input tensor, found {sorted(set(inputs))}")
        self.input_name = inputs[0]
        consumed = {t for ts in consumes.values() for t in ts}
        outs = [t for t in produced if t not in consumed]
        if len(outs) != 1:
            raise SEngineError(f"expected one graph output tensor, found {sorted(outs)}")
        self.output_name = outs[0]

        # buffer classes: spike tensors as bits, dense conv outputs as fp32 NHWC
        def cls(t):
            N, C, H, W = shapes[t]
            if self._is_real(t):
                return ("f32", N * H * W * C)
            if C % 32:
                raise SEngineError(f"tensor {t}: {C} channels is not a multiple of 32 (spike bits)")
            return ("bits", N * H * W * C // 32)

        self._producer_kind = {}
        for nid in self.schedule:
            self._producer_kind[self.ir.nodes[nid].output_names[0]] = _kname(self.ir.nodes[nid])
        sizes = {t: cls(t) for t in shapes}
        plan = plan_buffers(self.schedule, produces, consumes, aliases, sizes, {self.input_name, self.output_name})
        n_buf = 1 + max(b for b in plan.values() if b is not None)
        bufcls = {}
        for t, b in plan.items():
            if b is not None:
                bufcls[b] = sizes[t]
        self.buffers = [torch.empty(n, dtype=torch.float32 if k == "f32" else torch.int32, device=self.dev)
                        for k, n in (bufcls[i] for i in range(n_buf))]
        self.tensors = {}
        for t, b in plan.items():
            N, C, H, W = shapes[t]
            if b is None:
                continue
            last = C if self._is_real(t) else C // 32
            self.tensors[t] = self.buffers[b][: N * H * W * last].view(N, H, W, last)
        Ni, Ci, Hi, Wi = shapes[self.input_name]
        self._graph_input = torch.zeros(Ni, Hi, Wi, Ci, dtype=torch.float16, device=self.dev)
        No, Co, Ho, Wo = shapes[self.output_name]
        self._graph_output = torch.empty(No, Ho, Wo, Co, dtype=torch.float16, device=self.dev)
        self._shapes = shapes

        # weights, BN vectors, membranes
        for nid in self.schedule:
            node = ir.nodes[nid]
            name = _kname(node)
            if name in FUSED_VARIANTS or name in DENSE_VARIANTS:
                w = torch.from_numpy(np.ascontiguousarray(ir.weights[node.weight_info.name]))
                self.weights[nid] = self.kernels[nid].prepare_weight(w.to(self.dev), device=self.dev)
                self.bn[nid] = (torch.tensor(node.bn_scale, dtype=torch.float32, device=self.dev),
                                torch.tensor(node.bn_bias, dtype=torch.float32, device=self.dev))
                if keep_membranes and name in FUSED_VARIANTS:
                    N, C, H, W = node.output_shapes[0]
                    self.membranes[nid] = torch.zeros(N // self.T * H * W, C, device=self.dev)
            elif name in NEURON_VARIANTS and keep_membranes:
                N, C, H, W = node.output_shapes[0]
                self.membranes[nid] = torch.zeros(N // self.T * H * W * C, device=self.dev)
        self.graph = None
        return self

    def _is_real(self, t: str) -> bool:
        return self._producer_kind.get(t) in DENSE_VARIANTS

    # ------------------------------------------------------------------ execution
    def _execute_schedule(self):
        ops.pack_spikes(self._graph_input, out=self.tensors[self.input_name])  # first op of the graph
        for nid in self.schedule:
            node = self.ir.nodes[nid]
            name = _kname(node)
            if name == "ZeroCost":
                continue
            x = self.tensors[node.input_names[0]]
            y = self.tensors[node.output_names[0]]
            if name in FUSED_VARIANTS:
                sc, bi = self.bn[nid]
                mem = self.membranes.get(nid)
                args = (x, self.weights[nid], mem, sc, bi) if mem is not None else (x, self.weights[nid], sc, bi)
                self.kernels[nid](*args, out_enc=ENC_BITS, out=y)
            elif name in DENSE_VARIANTS:
                sc, bi = self.bn[nid]
                self.kernels[nid](x, self.weights[nid], sc, bi, out=y)
            else:  # standalone neuron on a dense conv's fp32 output
                p = node.neuron_params
                kind = "lif" if node.op_type.name == "LIF" else "if"
                v_reset = float(p.v_reset) if p.hard_reset else None
                ops.multistep_neuron(x.view(-1), self.T, kind, float(p.tau), float(p.v_threshold), v_reset,
                                     state=self.membranes.get(nid), out_enc=ENC_BITS, out=y.view(-1))
        ops.unpack_spikes(self.tensors[self.output_name], self._graph_output.shape[-1], out=self._graph_output)

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

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        """x: spikes (B, C, H, W) (repeated over T, as the reference's static-image input) or
        (T*B, C, H, W) NCHW, or (T*B, H, W, C) NHWC.  Returns fp16 NHWC spikes (T*B, OH, OW, C)."""
        TB, H, W, C = self._graph_input.shape
        if tuple(x.shape) != (TB, H, W, C):  # NCHW, per image (repeated over T) or per (t, b)
            if x.ndim != 4 or tuple(x.shape[1:]) != (C, H, W) or x.shape[0] not in (self.B, TB):
                raise SEngineError(f"input shape {tuple(x.shape)}: expected NHWC {(TB, H, W, C)} or NCHW "
                                   f"({self.B} or {TB}, {C}, {H}, {W})")
            if x.shape[0] != TB:
                x = x.repeat(self.T, 1, 1, 1)
            x = x.permute(0, 2, 3, 1)
        self._graph_input.copy_(x)
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
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n_iters):
            run()
        b.record()
        torch.cuda.synchronize(self.dev)
        return a.elapsed_time(b) / n_iters


HipGraphEngine = CUDAGraphEngine
