"""Numpy restatement of the data formats consumed by the gfx950 kernels.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  These formats are new in this
build (the reference keeps fp16 NHWC activations and dense (KH,KW,C_in,C_out)
weights, sengine/cuda_graph_runtime.py:202-249), so they are pinned by round trips
and known-answer placements, not by reference vectors.

Spike bits: (n_pos, C) -> uint32 (n_pos, C/32), channel c at bit c%32 of word c/32.

Sparse blob (v_smfmac_f32_16x16x64_f16 A operand), K_red ordered (kh, kw, c_in):
  values[G][q][plane][a][lane][8] fp16, meta[G][q][lane][a] uint32 (low 16 bits)
  lane l of tile a holds row r = l%16 <-> output channel 64G + 16*(r//4) + 4a + r%4,
  reduction indices 64q + 16*(l//16) + [0,16): four 4-groups, two kept values each,
  value j's in-group position in meta bits [2j+1:2j].
Dense blob (v_mfma_f32_16x16x32_f16 A operand): values[G][q32][plane][a][lane][8],
  lane l holds row r (same permutation), reduction indices 32q + 8*(l//16) + [0,8).
"""
from __future__ import annotations

import numpy as np

ZERO_TOL = 1e-10  # sengine/optimizer.py:522


def pack_bits(x: np.ndarray) -> np.ndarray:
    """(n_pos, C) values -> uint32 (n_pos, C//32); bit set where value != 0."""
    x = np.asarray(x)
    n, C = x.shape
    assert C % 32 == 0
    b = (x != 0).astype(np.uint64).reshape(n, C // 32, 32)
    words = (b << np.arange(32, dtype=np.uint64)).sum(axis=2)
    return words.astype(np.uint32)


def unpack_bits(words: np.ndarray, C: int) -> np.ndarray:
    """uint32 (n_pos, C//32) -> float32 (n_pos, C) of 0/1."""
    w = np.asarray(words, np.uint32)
    n = w.shape[0]
    bits = (w[:, :, None] >> np.arange(32, dtype=np.uint32)) & 1
    return bits.reshape(n, C).astype(np.float32)


def seq_to_nhwc_bits(x_seq: np.ndarray) -> np.ndarray:
    """(T, B, C, H, W) spikes -> packed (T*B*H*W, C/32) NHWC bits."""
    T, B, C, H, W = x_seq.shape
    nhwc = np.ascontiguousarray(np.transpose(x_seq, (0, 1, 3, 4, 2))).reshape(T * B * H * W, C)
    return pack_bits(nhwc)


def nhwc_bits_to_seq(words: np.ndarray, T, B, C, H, W) -> np.ndarray:
    x = unpack_bits(words, C).reshape(T, B, H, W, C)
    return np.ascontiguousarray(np.transpose(x, (0, 1, 4, 2, 3)))


def seq_to_planes(x_seq: np.ndarray, planes: int) -> np.ndarray:
    """Integer activations (T, B, C, H, W), values 0 .. 2^planes - 1 -> packed NHWC bit planes
    (T*B*H*W, planes*C/32): channel p*C + c holds bit p of channel c (the layout of the SEW
    residual output)."""
    x = np.asarray(x_seq).astype(np.int64)
    assert x.min() >= 0 and x.max() < (1 << planes)
    stacked = np.concatenate([(x >> p) & 1 for p in range(planes)], axis=2)
    return seq_to_nhwc_bits(stacked)


def planes_to_seq(words: np.ndarray, planes: int, T, B, C, H, W) -> np.ndarray:
    """Inverse of seq_to_planes: (T*B*H*W, planes*C/32) -> integer (T, B, C, H, W) float32."""
    x = nhwc_bits_to_seq(words, T, B, planes * C, H, W)
    return sum(x[:, :, p * C:(p + 1) * C] * float(1 << p) for p in range(planes)).astype(np.float32)


def _row_to_channel(G: int, a: int, r: np.ndarray) -> np.ndarray:
    return 64 * G + 16 * (r // 4) + 4 * a + (r % 4)


def _planes(kept: np.ndarray, planes: int) -> np.ndarray:
    hi = kept.astype(np.float16)
    if planes == 1:
        return hi[None]
    lo = (kept.astype(np.float32) - hi.astype(np.float32)).astype(np.float16)
    return np.stack([hi, lo])


def compress_2_4(w: np.ndarray, planes: int = 1):
    """OIHW weight (C_out, C_in, KH, KW) -> (values uint16, meta uint32, violations int32).

    A 4-group keeps its entries with |w| >= 1e-10 (at most two; extra ones are a
    violation and are dropped after the first two), padded with the lowest unused
    positions holding 0; kept positions ascending.
    """
    w = np.asarray(w)
    C_out, C_in, KH, KW = w.shape
    assert C_in % 64 == 0 and C_out % 64 == 0
    wf = w.astype(np.float32)
    # reduction-major view: (C_out, K_red) with K_red ordered (kh, kw, c_in)
    wk = np.transpose(wf, (0, 2, 3, 1)).reshape(C_out, KH * KW * C_in)
    K_red = wk.shape[1]
    nq, nG = K_red // 64, C_out // 64
    groups = wk.reshape(C_out, K_red // 4, 4)
    keep = np.abs(groups) >= ZERO_TOL
    n_keep = keep.sum(axis=2)
    violations = (n_keep > 2).astype(np.int32)  # (C_out, K_red/4) == ((co,kh,kw), c/4) order
    # kept entries first (in index order), then the unused positions in index order
    key = np.where(keep, 0, 4) + np.arange(4)
    pos = np.sort(np.argsort(key, axis=2, kind="stable")[..., :2], axis=2)
    vals = np.take_along_axis(groups, pos, axis=2)
    vals = np.where(np.abs(vals) >= ZERO_TOL, vals, 0.0).astype(np.float32)
    # vals: (C_out, K_red/4, 2); meta bits per group: pos0 | pos1 << 2
    gbits = (pos[..., 0] | (pos[..., 1] << 2)).astype(np.uint32)
    values = np.zeros((nG, nq, planes, 4, 64, 8), np.float16)
    meta = np.zeros((nG, nq, 64, 4), np.uint32)
    lanes = np.arange(64)
    r = lanes % 16
    for G in range(nG):
        for a in range(4):
            co = _row_to_channel(G, a, r)  # (64,)
            for q in range(nq):
                g0 = (64 * q + 16 * (lanes // 16)) // 4  # first 4-group index per lane
                gidx = g0[:, None] + np.arange(4)[None, :]  # (64, 4)
                v = vals[co[:, None], gidx]  # (64, 4, 2)
                values[G, q, :, a] = _planes(v.reshape(64, 8), planes)
                bits = gbits[co[:, None], gidx]  # (64, 4)
                m = np.zeros(64, np.uint32)
                for gi in range(4):
                    m |= bits[:, gi] << np.uint32(4 * gi)
                meta[G, q, :, a] = m
    return values.view(np.uint16), meta, violations.reshape(-1)


def flat_weight(w: np.ndarray, H: int, W: int, stride: int = 1, padding: int = 0, dilation: int = 1) -> np.ndarray:
    """The flat small-output layout of this build's library: an OIHW conv weight
    (C_out, C_in, KH, KW) applied to H x W inputs as one matrix (N_flat, K_flat, 1, 1) with
    rows (oh, ow, c_out) and reduction (ih, iw, c_in) -- NHWC order on both sides -- holding
    w[f, c, kh, kw] where input pixel (ih, iw) meets output pixel (oh, ow) through tap
    (kh, kw), and 0 elsewhere.  conv2d(x, w) == x_nhwc_flat @ flat.T (pinned against
    torch.nn.functional.conv2d in tests/test_oracle.py)."""
    w = np.asarray(w)
    C_out, C_in, KH, KW = w.shape
    OH = (H + 2 * padding - dilation * (KH - 1) - 1) // stride + 1
    OW = (W + 2 * padding - dilation * (KW - 1) - 1) // stride + 1
    flat = np.zeros((OH, OW, C_out, H, W, C_in), w.dtype)
    for oh in range(OH):
        for ow in range(OW):
            for kh in range(KH):
                for kw in range(KW):
                    ih = oh * stride - padding + kh * dilation
                    iw = ow * stride - padding + kw * dilation
                    if 0 <= ih < H and 0 <= iw < W:
                        flat[oh, ow, :, ih, iw, :] = w[:, :, kh, kw]
    return flat.reshape(OH * OW * C_out, H * W * C_in, 1, 1)


def decompress_2_4(values: np.ndarray, meta: np.ndarray, shape) -> np.ndarray:
    """Inverse of compress_2_4 (planes summed in fp32) -> OIHW float32."""
    C_out, C_in, KH, KW = shape
    vals = np.asarray(values).view(np.float16).astype(np.float32).sum(axis=2)  # (nG,nq,4,64,8)
    nG, nq = vals.shape[0], vals.shape[1]
    wk = np.zeros((C_out, KH * KW * C_in), np.float32)
    lanes = np.arange(64)
    r = lanes % 16
    for G in range(nG):
        for a in range(4):
            co = _row_to_channel(G, a, r)
            for q in range(nq):
                m = meta[G, q, :, a]
                for j in range(8):
                    gi = j // 2
                    p = (m >> np.uint32(2 * j)) & 3
                    k = 64 * q + 16 * (lanes // 16) + 4 * gi + p.astype(np.int64)
                    np.add.at(wk, (co, k), vals[G, q, a, :, j])
    return np.ascontiguousarray(np.transpose(wk.reshape(C_out, KH, KW, C_in), (0, 3, 1, 2)))


def pack_dense(w: np.ndarray, planes: int = 1) -> np.ndarray:
    """OIHW weight -> dense blob values (uint16 view of fp16)."""
    w = np.asarray(w).astype(np.float32)
    C_out, C_in, KH, KW = w.shape
    assert C_in % 32 == 0 and C_out % 64 == 0
    wk = np.transpose(w, (0, 2, 3, 1)).reshape(C_out, KH * KW * C_in)
    nq, nG = wk.shape[1] // 32, C_out // 64
    values = np.zeros((nG, nq, planes, 4, 64, 8), np.float16)
    lanes = np.arange(64)
    r = lanes % 16
    for G in range(nG):
        for a in range(4):
            co = _row_to_channel(G, a, r)
            for q in range(nq):
                k = 32 * q + 8 * (lanes // 16)
                v = wk[co[:, None], k[:, None] + np.arange(8)[None, :]]
                values[G, q, :, a] = _planes(v, planes)
    return values.view(np.uint16)


def unpack_dense(values: np.ndarray, shape) -> np.ndarray:
    C_out, C_in, KH, KW = shape
    vals = np.asarray(values).view(np.float16).astype(np.float32).sum(axis=2)
    nG, nq = vals.shape[0], vals.shape[1]
    wk = np.zeros((C_out, KH * KW * C_in), np.float32)
    lanes = np.arange(64)
    r = lanes % 16
    for G in range(nG):
        for a in range(4):
            co = _row_to_channel(G, a, r)
            for q in range(nq):
                k = 32 * q + 8 * (lanes // 16)
                wk[co[:, None], k[:, None] + np.arange(8)[None, :]] = vals[G, q, a]
    return np.ascontiguousarray(np.transpose(wk.reshape(C_out, KH, KW, C_in), (0, 3, 1, 2)))
