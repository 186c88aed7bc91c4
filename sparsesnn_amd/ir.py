"""Graph-node contract of the fused operator (the part of sengine/ir.py this path uses).

The enum member names and node fields are the reference's interface (sengine/ir.py:16-269):
the graph passes, fusion strategy and runtime address kernels by these names, so a node
built by the reference's own parser/optimizer is accepted as-is (the compiler in
sparsesnn_amd/compiler.py matches enums by *name* and reads nodes by attribute).  The
IR below is a small self-contained implementation for building and testing such graphs
without the reference.
"""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
from enum import Enum, auto
from typing import Optional


class OpType(Enum):
    Conv2d = auto()
    Linear = auto()
    LIF = auto()
    IF = auto()
    MS = auto()
    Add = auto()
    BatchNorm = auto()
    Reshape = auto()
    Transpose = auto()
    Identity = auto()
    Flatten = auto()
    MaxPool = auto()
    GlobalAvgPool = auto()
    Tile = auto()            # repeat over T (the static image fed to every timestep)
    TemporalMean = auto()
    Gemm = auto()            # classifier Linear
    FusedAttention = auto()  # attention core (q, k, v spikes -> attention neuron spikes), one custom node


class NeuronType(Enum):
    LIF = auto()
    IF = auto()
    MS = auto()
    NoNeuron = auto()


class KernelVariant(Enum):
    """Kernel choices for a node (names as in sengine/ir.py:51-95).

    FusedSparseConvBNLIF: declared but never compiled by the reference
    (sengine/optimizer.py:845-848 assigns it, tilelang_compiler.py:427-481 has no branch);
    here it is the gfx950 2:4 SMFMAC kernel.  TileLangFusedConvBNIF / TileLangFusedConv1x1BNIF
    (the reference's dense fused nodes) are served by the same kernel when the weights are
    2:4, otherwise by the dense fallback.  TileLangConvBN / TileLangConv1x1BN + CUDAVec4LIF /
    CUDAVec4IF / StandaloneLIF are the unfused fallback halves.  TileLangStemConvBN,
    CuDNNPool, Elementwise, TemporalMean, TileRepeat and CuBLASGemm are the network-level
    node kinds around the fused op (sengine/cuda_graph_runtime.py:819-880); the passes in
    sparsesnn_amd/passes.py absorb them into fused launches where the kernels allow.
    """
    CuDNNConv = auto()
    FusedSparseConvBNLIF = auto()
    StandaloneLIF = auto()
    ZeroCost = auto()
    TileLangConvBN = auto()
    TileLangConv1x1BN = auto()
    CUDAVec4IF = auto()
    CUDAVec4LIF = auto()
    TileLangFusedConvBNIF = auto()
    TileLangFusedConv1x1BNIF = auto()
    TileLangStemConvBN = auto()   # dense C_in=3 stem conv + BN on the images
    CuDNNPool = auto()            # MaxPool / GlobalAvgPool
    Elementwise = auto()          # Add
    TemporalMean = auto()
    TileRepeat = auto()
    CuBLASGemm = auto()           # classifier
    FusedSpikformerAttn = auto()  # Spikformer SSA core: (Q K^T * scale) V per head -> attention LIF


class BoundType(Enum):
    COMPUTE = "C"
    MEMORY = "M"
    ZERO = "Z"


class TensorLayout(Enum):
    NCHW = auto()
    NHWC = auto()
    ND = auto()


@dataclass
class KernelLayoutContract:
    input_layout: TensorLayout
    output_layout: TensorLayout


# Layout contracts of the variants this path serves (sengine/ir.py:135-176): conv kernels
# are NHWC -> NHWC; neuron kernels inherit their predecessor's layout (None).
KERNEL_CONTRACTS = {
    KernelVariant.FusedSparseConvBNLIF: KernelLayoutContract(TensorLayout.NHWC, TensorLayout.NHWC),
    KernelVariant.TileLangFusedConvBNIF: KernelLayoutContract(TensorLayout.NHWC, TensorLayout.NHWC),
    KernelVariant.TileLangFusedConv1x1BNIF: KernelLayoutContract(TensorLayout.NHWC, TensorLayout.NHWC),
    KernelVariant.TileLangConvBN: KernelLayoutContract(TensorLayout.NHWC, TensorLayout.NHWC),
    KernelVariant.TileLangConv1x1BN: KernelLayoutContract(TensorLayout.NHWC, TensorLayout.NHWC),
    KernelVariant.CuDNNConv: KernelLayoutContract(TensorLayout.NHWC, TensorLayout.NHWC),
    KernelVariant.CUDAVec4IF: None,
    KernelVariant.CUDAVec4LIF: None,
    KernelVariant.StandaloneLIF: None,
    KernelVariant.ZeroCost: None,
    KernelVariant.TileLangStemConvBN: KernelLayoutContract(TensorLayout.NCHW, TensorLayout.NHWC),
    KernelVariant.CuDNNPool: KernelLayoutContract(TensorLayout.NHWC, TensorLayout.NHWC),
    KernelVariant.Elementwise: None,
    KernelVariant.TemporalMean: None,
    KernelVariant.TileRepeat: None,
    KernelVariant.CuBLASGemm: KernelLayoutContract(TensorLayout.ND, TensorLayout.ND),
    KernelVariant.FusedSpikformerAttn: KernelLayoutContract(TensorLayout.NHWC, TensorLayout.NHWC),
}


@dataclass
class ConvParams:
    in_channels: int = 0
    out_channels: int = 0
    kernel_h: int = 1
    kernel_w: int = 1
    stride_h: int = 1
    stride_w: int = 1
    pad_h: int = 0
    pad_w: int = 0
    dilation_h: int = 1
    dilation_w: int = 1
    groups: int = 1


@dataclass
class NeuronParams:
    neuron_type: NeuronType = NeuronType.NoNeuron
    T: int = 4
    tau: float = 1.0
    v_threshold: float = 1.0
    v_reset: float = 0.0
    hard_reset: bool = True


@dataclass
class AttentionParams:
    """Attention-core node parameters (sengine/ir.py:205-215): the variant, head geometry, the
    product's scale and the attention neuron (a LIF, hard reset to 0)."""
    variant: str = ""
    num_heads: int = 1
    head_dim: int = 64
    scale: float = 1.0
    H: int = 0
    W: int = 0
    attn_lif_tau: float = 2.0
    attn_lif_v_threshold: float = 1.0


@dataclass
class WeightInfo:
    name: str = ""
    shape: tuple = ()
    is_sparse: bool = False
    onnx_idx: int = -1


@dataclass
class Node:
    id: int
    name: str
    op_type: OpType
    is_stateful: bool = False
    input_names: list = field(default_factory=list)
    output_names: list = field(default_factory=list)
    input_shapes: list = field(default_factory=list)   # NCHW with N = T*B, as the reference
    output_shapes: list = field(default_factory=list)
    conv_params: Optional[ConvParams] = None
    neuron_params: Optional[NeuronParams] = None
    pool_params: Optional[dict] = None    # kernel_size / stride / padding (MaxPool)
    gemm_params: Optional[dict] = None
    attention_params: Optional[AttentionParams] = None
    extra_attrs: dict = field(default_factory=dict)
    assigned_kernel: KernelVariant = KernelVariant.ZeroCost
    layout: TensorLayout = TensorLayout.NCHW
    fusion_group_id: int = -1
    sparse_weight: bool = False
    weight_info: Optional[WeightInfo] = None
    bias_info: Optional[WeightInfo] = None
    bn_scale: Optional[list] = None
    bn_bias: Optional[list] = None
    bound_type: BoundType = BoundType.ZERO
    tilelang_config: Optional[dict] = None
    est_latency_us: float = 0.0


@dataclass
class FusionGroup:
    group_id: int
    conv_node_id: int
    bn_node_id: int = -1
    neuron_node_id: int = -1
    variant: KernelVariant = KernelVariant.FusedSparseConvBNLIF
    bn_scale: Optional[list] = None
    bn_bias: Optional[list] = None


class EngineIR:
    """DAG of nodes connected by tensor names (producer/consumer maps)."""

    def __init__(self):
        self.nodes: dict = {}
        self.fusion_groups: list = []
        self.T: int = 4
        self.precision: str = "fp16"
        self.weights: dict = {}          # name -> numpy array (OIHW conv weights, BN vectors)
        self._producer: dict = {}
        self._consumers: dict = {}
        self._next_id = 0
        self._topo: list = []

    def add_node(self, node: Node) -> int:
        nid = self._next_id
        self._next_id += 1
        node.id = nid
        self.nodes[nid] = node
        for o in node.output_names:
            self._producer[o] = nid
        for i in node.input_names:
            self._consumers.setdefault(i, []).append(nid)
        self._topo = []
        return nid

    def predecessors(self, nid: int) -> list:
        out = []
        for i in self.nodes[nid].input_names:
            p = self._producer.get(i)
            if p is not None and p in self.nodes and p not in out:
                out.append(p)
        return out

    def successors(self, nid: int) -> list:
        out = []
        for o in self.nodes[nid].output_names:
            for c in self._consumers.get(o, []):
                if c in self.nodes and c not in out:
                    out.append(c)
        return out

    @property
    def topo_order(self) -> list:
        if not self._topo:
            indeg = {n: len(self.predecessors(n)) for n in self.nodes}
            q = deque(sorted(n for n, d in indeg.items() if d == 0))
            order = []
            while q:
                n = q.popleft()
                order.append(n)
                for s in self.successors(n):
                    indeg[s] -= 1
                    if indeg[s] == 0:
                        q.append(s)
            if len(order) != len(self.nodes):
                raise ValueError("graph has a cycle")
            self._topo = order
        return self._topo

    def remove_node(self, nid: int):
        """Remove a single-input pass-through node (e.g. a folded BN): its consumers are
        rewired to its data input."""
        node = self.nodes.pop(nid)
        src = node.input_names[0] if node.input_names else None
        for o in node.output_names:
            for c in self._consumers.pop(o, []):
                if c in self.nodes and src is not None:
                    cn = self.nodes[c]
                    cn.input_names = [src if x == o else x for x in cn.input_names]
                    self._consumers.setdefault(src, []).append(c)
            if self._producer.get(o) == nid:
                del self._producer[o]
        for i in node.input_names:
            if i in self._consumers:
                self._consumers[i] = [c for c in self._consumers[i] if c != nid]
        self._topo = []
