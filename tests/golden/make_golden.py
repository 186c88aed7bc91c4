"""Writes tests/golden/cfg0_golden.npz: BASELINE.json config 0 through the CPU oracle.

Config 0: T=4, batch 1, spikes ~ Bernoulli(0.15) of shape (4, 1, 64, 32, 32); conv 3x3
64->64 stride 1 pad 1, fp32 weights ~ N(0, 2/(9*64)) with a 2:4 magnitude mask along
input channels; BN gamma ~ U(0.5,1.5), beta ~ N(0,0.1), mean ~ N(0,0.1), var ~ U(0.5,1.5),
eps 1e-5; LIF tau=2, V_th=1, hard reset to 0, V0=0.  Seed 0, draw order as in
oracle.reference_path.make_layer_case.

The reference holds no vectors of its own for this path (no tests, no stored outputs),
so the fixture is produced by the oracle, whose functions are pinned independently in
tests/test_oracle.py.  It stores the packed input spikes, the fp32 weights, the BN
parameters, the expected output spikes (packed, NHWC bit order) and the charged membrane
per timestep (fp32, NCHW).  Usage: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import packing as pk  # noqa: E402
from oracle import reference_path as ref  # noqa: E402

CFG0 = dict(seed=0, T=4, B=1, C_in=64, C_out=64, H=32, W=32, k=3)


def make(path=os.path.join(HERE, "cfg0_golden.npz")):
    c = ref.make_layer_case(CFG0["seed"], T=4, B=1, C_in=64, C_out=64, H=32, W=32, k=3)
    r = ref.fused_layer(c.x_seq, c.w, c.bn, c.stride, c.padding, 1, "lif", 2.0, 1.0, 0.0)
    x_bits = pk.seq_to_nhwc_bits(c.x_seq.numpy())
    s_bits = pk.seq_to_nhwc_bits(r.spikes.numpy())
    np.savez_compressed(
        path, x_bits=x_bits, w=c.w.numpy(), gamma=c.bn.gamma.numpy(), beta=c.bn.beta.numpy(),
        mean=c.bn.mean.numpy(), var=c.bn.var.numpy(), eps=np.float32(c.bn.eps), spikes_bits=s_bits,
        h=r.h.numpy().astype(np.float32), shape=np.array([4, 1, 64, 32, 32, 64, 3, 1, 1]),
        lif=np.array([2.0, 1.0, 0.0], np.float32))
    return path


if __name__ == "__main__":
    print(make())
