"""GPU: the allocation-free attention entry (sengine_amd_ssa_attention_noalloc) through the C
ABI against the workspace entries (sengine_amd_ssa_kv + sengine_amd_ssa_attend_neuron) on the
same inputs: bit-identical spikes on two calls in a row, the second smaller (the library's
array keeps the first call's contents), and the size limit refused before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from sparsesnn_amd import _lib, ops

pytestmark = pytest.mark.gpu

NEURON_LIF = 0


def _bits(dev, T, B, N, C, p, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand((T * B, N, C), generator=g) < p).half().to(dev)
    return ops.pack_spikes(x)


def _noalloc(dev, q, k, v, T, B, N, C, heads, scale=0.125):
    out = torch.full((T * B, N, C // 32), -1, dtype=torch.int32, device=dev)
    rc = _lib.load().sengine_amd_ssa_attention_noalloc(T, B, N, C, heads, scale, NEURON_LIF, 1, 2.0, 0.5, 0.0,
                                                       q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                                       torch.cuda.current_stream(dev).cuda_stream)
    return rc, out


def test_noalloc_attention_matches_workspace_entries(dev):
    for (T, B, N, C, heads, seed) in ((4, 2, 700, 384, 8, 1), (2, 1, 130, 128, 2, 2)):  # second call smaller
        q, k, v = (_bits(dev, T, B, N, C, 0.25, seed * 10 + i) for i in range(3))
        ref = ops.spiking_self_attention(q, k, v, T, B, N, C, heads)
        rc, got = _noalloc(dev, q, k, v, T, B, N, C, heads)
        torch.cuda.synchronize()
        assert rc == 0, _lib.load().sengine_amd_last_error().decode()
        assert torch.equal(got, ref), int((got != ref).sum())
        assert float(ops.unpack_spikes(ref, C).float().mean()) > 0.01


def test_noalloc_attention_refuses_oversize(dev):
    T, B, N, C, heads = 8, 128, 16, 512, 8  # 8 * 128 * 8 * 64^2 = 33.5M entries > 4M
    z = torch.zeros(T * B * N * C // 32, dtype=torch.int32, device=dev)
    rc, _ = _noalloc(dev, z, z, z, T, B, N, C, heads)
    assert rc == -2
    assert "scratch" in _lib.load().sengine_amd_last_error().decode()
