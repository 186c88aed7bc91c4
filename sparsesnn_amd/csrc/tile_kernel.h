// Fused 2:4-sparse Conv + BN + multi-step LIF/IF for spike-bit inputs, with the spikes
// expanded to fp16 once per workgroup in LDS ("tile" kernels; gfx950 fast path).
//
// Same operator, GEMM view and weight blob as fused_sparse.hip / fused_sparse_lds.hip
// (the reference's conv2d_bn_if_interleaved_kernel and conv1x1_bn_lif,
// sengine/kernels/conv2d_bn_if_t4.py:918-1022, interleaved_templates.py:95-154).
//
// On the MI355X the v_smfmac_f32_16x16x64_f16 issue rate is limited less by the
// matrix cores than by everything else the SIMD must do per SMFMAC: VALU ops (~4 cycles
// each, not overlapped with the SMFMAC) and operand bytes returned into VGPRs by LDS
// and global loads (~16 cycles per KB per SIMD, measured).  The design minimises both:
//
//  * The spike bits are expanded to fp16 (value 2.0, factor 1/2 folded into the BN scale)
//    once per workgroup and input pixel, into LDS, instead of once per wave, tap and
//    fragment: a B fragment is then two ds_read_b128 (channels 8g..8g+7 and
//    32+8g..32+8g+7 of the pixel) and no VALU.
//  * KS == 3 (3x3, stride 1, pad 1): a workgroup owns a TR x TC tile of output pixels of
//    one image; LDS holds the (TR+2) x (TC+2) halo of input pixels, so the 9 taps are
//    compile-time offsets from a per-lane base and every input pixel is expanded once,
//    not 9 times.  Each wave owns a GR-row x 2-column block of the tile (lane column l is
//    block pixel (l/2, l%2)); with a halo row length HC = 2 (mod 4) (or GR = 7, HC = 9)
//    the 16 pixels of a block land in 16 distinct 16-byte bank groups for every tap.
//  * KS == 0 (fp16 input, any kernel size / stride / padding / dilation: the reference ABI's
//    activations on geometries the other forms do not cover): like KS == 1, but the reduction
//    runs over the KH*KW*C_in/64 chunks of the blob, and chunk q stages, for each (t, position),
//    the 64 fp16 channels of the input pixel under tap q / (C_in/64) (zero in the padding):
//    an implicit im2col, one tap per chunk, with the same LDS layout and loop.
//  * KS == 1 (1x1, any stride, pad 0): a workgroup owns 64 consecutive output positions
//    (flattened b, oh, ow); LDS holds their input pixels, double-buffered across the
//    64-channel reduction chunks (one barrier per chunk).
//  * A wave owns 16 positions x 64*GPW output channels x all T: T*4*GPW accumulator tiles
//    in VGPRs, so the LIF recurrence over t runs in registers (the membrane never touches
//    HBM).  GPW = 2 halves the B bytes per SMFMAC (each fragment feeds 8 SMFMACs).
//  * A operands (2:4 values + metadata) come from global memory (L2-resident, shared by
//    every workgroup of a channel group), one tap ahead of their use.
//  * LDS layout: 8-byte half-pieces; half-piece q = 8h + i (piece i holds channels
//    8i..8i+7, half h channels 8i+4h..8i+4h+3) of pixel px at timestep t sits at entry
//    t*(16*NPIX + PAD) + (q >> 1)*NPIX + (q & 1)*(8*NPIX + PAD) + px: even and odd q in
//    two regions, the odd one PAD entries further on.  Staging writes are consecutive and
//    a fragment is four 8-byte reads (measured cheaper for the SIMD than two 16-byte
//    reads).  The LDS has 64 four-byte banks and serves a ds_read_b64 32 lanes at a time,
//    i.e. lane groups g, g+1 that read half-pieces q, q+1 of the same pixels; PAD (per tile
//    shape, found by enumerating the banks of every fragment read of the shape) puts the two
//    groups on disjoint banks, and lanes outside the tile read the address of a lane inside
//    it (same address: broadcast).  Without the shift the same reads measured 1.45x the
//    LDS cycles.
//  * Workgroup ids are remapped so each XCD (own L2) runs a contiguous range of
//    (channel block, tile) ids: an XCD touches few channel blocks' weights.
#pragma once
#include "common.h"
#include "epilogue.h"
#include "internal.h"

namespace sengine {

struct TileParams {
  const uint8_t* in;
  const u32x4_t* wvals;
  const uint32_t* wmeta;
  float* state;
  const float* scale;
  const float* bias;
  uint8_t* out;
  float* h_trace;
  float* x_trace;
  int B, C, H, W, F, OH, OW, S;  // S: stride (KS == 1 only)
  int KW, SH, SW, PH, PW, DH, DW;  // KS == 0: kernel width, strides, paddings, dilations
  int M;                         // B*OH*OW positions per timestep
  int nchunk;                    // C / 64
  int nq;                        // KH*KW*nchunk reduction chunks in the blob
  int tiles_w, tiles_per_image;  // KS == 3: spatial tiles
  int ntiles;                    // tiles per channel block
  NeuronParams np;
  float enc_scale;
  SewAdd sew;
};

template <int KS, int TR, int TC, int GR>
struct TileGeom {
  static constexpr int HC = KS == 3 ? TC + 2 : 0;
  static constexpr int NPIX = KS == 3 ? (TR + 2) * (TC + 2) : 64;
  static constexpr int NCP = KS == 3 ? (TC + 1) / 2 : 1;
  static constexpr int NWAVE = KS == 3 ? NCP * ((TR + GR - 1) / GR) : 4;
  static constexpr int NTHR = 64 * NWAVE;
  static constexpr int NTAP = KS == 0 ? 1 : KS * KS;  // taps per chunk
  static constexpr int NBUF = KS == 3 ? 1 : 2;
  // odd half-piece region shift (entries) that makes every fragment read conflict-free
  static constexpr int PAD = (KS == 3 && TR == 7 && TC == 7) ? 8 : 16;
  static constexpr int TS = 16 * NPIX + PAD;  // entries per timestep
};

// Consecutive hardware workgroup ids go round-robin over the 8 XCDs; give XCD x the
// logical ids [x*per, (x+1)*per) instead (ragged tail unchanged).
__device__ __forceinline__ int tile_remap(int id, int n) {
  const int per = n >> 3;
  if (id >= per * 8) return id;
  return (id & 7) * per + (id >> 3);
}

// 64 spike bits (channel c = bit c) -> 64 fp16 values in 8 pieces of 8 channels.
__device__ __forceinline__ void expand_word64(uint2 w, u32x4_t (&pc)[8]) {
  const uint32_t parts[4] = {w.x & 0xffffu, w.x >> 16, w.y & 0xffffu, w.y >> 16};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const u32x8_t e = __builtin_bit_cast(u32x8_t, expand_bits16(parts[k]));
    pc[2 * k] = u32x4_t{e[0], e[1], e[2], e[3]};
    pc[2 * k + 1] = u32x4_t{e[4], e[5], e[6], e[7]};
  }
}

// KSP = 2 splits the reduction inside the workgroup: a second set of waves covers the same
// positions and channels over the odd reduction chunks (its own LDS buffer), and its
// accumulators are added to the first set's in LDS, in a fixed order, before the
// epilogue.  Twice the waves per tile for layers whose grid leaves SIMDs with one wave.
//
// The generic epilogue (any neuron, traces, the membrane-shortcut form) is allowed two waves
// per SIMD: its fp32 residual rows are loaded for all T at once.
//
// PF = 2 (3x3 only) prefetches A operands two taps and B fragments two (tap, t) steps
// ahead instead of one: for grids of at most two workgroups per CU, whose waves (two per
// SIMD) have the registers for it and whose SMFMAC issue otherwise waits on L2 and LDS
// latency.
//
// IN_ENC = SENGINE_ENC_F16 (the reference's fp16 NHWC activations, any fp16 values): each
// (t, pixel) unit of a chunk is 64 fp16 = eight 16-byte pieces, copied as they are into the
// same LDS half-piece layout (no expansion); a thread moves pieces tid, tid + NTHR, ... and
// the next chunk's pieces are loaded into registers when a chunk's reduction starts (up to
// ~52 registers: these instances run two waves per SIMD).
template <int T, int KS, int TR, int TC, int GR, int GPW, int OUT_ENC, int MODE, int KSP, int PF = 1,
          int IN_ENC = SENGINE_ENC_BITS>
__global__ __launch_bounds__((TileGeom<KS, TR, TC, GR>::NTHR * KSP))
__attribute__((amdgpu_waves_per_eu(GPW == 1 && KSP == 1 && PF == 1 && MODE != EPI_GENERIC && IN_ENC == SENGINE_ENC_BITS &&
                                           !(KS == 3 && OUT_ENC == SENGINE_ENC_F16)
                                       ? 3
                                       : (GPW == 2 && KS == 3 ? 1 : 2)))) void fused_tile_kernel(TileParams p) {
  using Gm = TileGeom<KS, TR, TC, GR>;
  static_assert(PF == 1 || (PF == 2 && KS == 3), "two-deep prefetch needs the unrolled 9-tap loop");
  static_assert(KS != 0 || (IN_ENC == SENGINE_ENC_F16 && KSP == 1), "the gather form stages fp16 rows");
  constexpr int NA = PF + 1;  // A operand sets in flight (ring over taps; 9 % 3 == 0)
  constexpr int NB = PF + 1;  // B fragment sets in flight (ring over (tap, t) steps)
  constexpr int NPIX = Gm::NPIX;
  constexpr int NTHR = Gm::NTHR;  // threads of one set
  constexpr int NTAP = Gm::NTAP;
  constexpr int NBUF = Gm::NBUF;
  constexpr int NCH = 64 * GPW;
  constexpr int UNITS = T * NPIX;                 // (t, pixel) spike words per chunk
  constexpr int UPT = (UNITS + NTHR - 1) / NTHR;  // per thread
  constexpr int PAD = Gm::PAD;
  constexpr int TS = Gm::TS;
  constexpr int BUFE = T * TS;  // entries per buffer
  __shared__ uint2 sB[NBUF * KSP][BUFE];
  __shared__ float sCoef[4][NCH];

  // wave-uniform (NTHR is a multiple of 64): keeps the reduction-chunk loop in scalar registers
  const int set = KSP == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)threadIdx.x / NTHR);
  const int tid = (int)threadIdx.x - set * NTHR;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int col = lane & 15;

  const int L = tile_remap(blockIdx.x, gridDim.x);
  // Bit input: channel-block-major ids (an XCD's workgroups share few blocks' weights).  fp16
  // input: tile-major ids, so the channel blocks of one tile run together on one XCD and read
  // its 16-bit activations from HBM once (the other blocks hit L2) instead of once per block.
  const int ncb = p.F / (64 * GPW);
  const int Gb = IN_ENC == SENGINE_ENC_F16 ? L % ncb : L / p.ntiles;  // channel block: groups Gb*GPW ..
  const int tile = IN_ENC == SENGINE_ENC_F16 ? L / ncb : L - Gb * p.ntiles;
  const int G0 = Gb * GPW;
  int b = 0, oh0 = 0, ow0 = 0, m0 = 0;
  if (KS == 3) {
    b = tile / p.tiles_per_image;
    const int trc = tile - b * p.tiles_per_image;
    const int tr = trc / p.tiles_w;
    oh0 = tr * TR;
    ow0 = (trc - tr * p.tiles_w) * TC;
  } else {
    m0 = tile * 64;
  }

  const bool fold = MODE == EPI_LIF_HARD || (MODE == EPI_GENERIC && p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2);
  if (set == 0 && tid < NCH) {
    const float sc = p.scale[G0 * 64 + tid] * p.enc_scale;  // exact: enc_scale is a power of two
    const float bi = p.bias[G0 * 64 + tid];
    sCoef[0][tid] = fold ? sc * p.np.rtau : sc;             // exact: rtau is a power of two
    sCoef[1][tid] = fold ? bi * p.np.rtau : bi;
    sCoef[2][tid] = sc;
    sCoef[3][tid] = bi;
  }

  // ---- staging identity: units u = tid + j*NTHR -> (t, pixel); goff -1 = zero word
  const int cbytes = p.C >> 3;
  int goff[UPT];  // byte offsets: the host guarantees the input spans < 2^31 bytes
  int soff[UPT];
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const int u = tid + j * NTHR;
    const int t = u / NPIX;
    const int px = u - t * NPIX;
    int ib = b, ih, iw;
    bool inb;
    if (KS == 3) {
      const int hr = px / Gm::HC;
      ih = oh0 - 1 + hr;
      iw = ow0 - 1 + (px - hr * Gm::HC);
      inb = u < UNITS && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W;
    } else {
      const int m = m0 + px;
      inb = u < UNITS && m < p.M;
      const int ohw = p.OH * p.OW;
      ib = inb ? m / ohw : 0;
      const int r = m - ib * ohw;
      const int oh = inb ? r / p.OW : 0;
      ih = oh * p.S;
      iw = (r - oh * p.OW) * p.S;
    }
    goff[j] = inb ? (((t * p.B + ib) * p.H + ih) * p.W + iw) * cbytes : -1;
    soff[j] = t * TS + px;
  }
  auto load_units = [&](uint2 (&v)[UPT], int c) {
#pragma unroll
    for (int j = 0; j < UPT; ++j)
      v[j] = goff[j] >= 0 ? *reinterpret_cast<const uint2*>(p.in + goff[j] + c * 8) : uint2{0u, 0u};
  };
  // fp16 input: 16-byte pieces; piece pc = tid + j*NTHR is piece pc & 7 of unit pc >> 3
  constexpr int PPT = IN_ENC == SENGINE_ENC_F16 ? (UNITS * 8 + NTHR - 1) / NTHR : 1;
  auto unit_off16 = [&](int u) {  // byte offset of unit u's fp16 pixel row, or -1 (zero)
    const int t = u / NPIX;
    const int px = u - t * NPIX;
    int ib = b, ih, iw;
    bool inb;
    if (KS == 3) {
      const int hr = px / Gm::HC;
      ih = oh0 - 1 + hr;
      iw = ow0 - 1 + (px - hr * Gm::HC);
      inb = u < UNITS && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W;
    } else {
      const int m = m0 + px;
      inb = u < UNITS && m < p.M;
      const int ohw = p.OH * p.OW;
      ib = inb ? m / ohw : 0;
      const int r = m - ib * ohw;
      const int oh = inb ? r / p.OW : 0;
      ih = oh * p.S;
      iw = (r - oh * p.OW) * p.S;
    }
    return inb ? (((t * p.B + ib) * p.H + ih) * p.W + iw) * (p.C * 2) : -1;
  };
  // byte offsets of this thread's pieces' fp16 rows (fixed over the chunks; -1 = zero piece).
  // KS == 0: instead the (t, image) row block of the piece's position (-1: past M) and the
  // top-left input pixel of its receptive field, ih0 in the high and iw0 in the low 16 bits.
  int off16[IN_ENC == SENGINE_ENC_F16 ? PPT : 1];
  int gpix[KS == 0 ? PPT : 1];
  if (IN_ENC == SENGINE_ENC_F16 && KS != 0) {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int pc = tid + j * NTHR;
      const int o = pc < UNITS * 8 ? unit_off16(pc >> 3) : -1;
      off16[j] = o < 0 ? -1 : o + (pc & 7) * 16;
    }
  }
  if (KS == 0) {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int u = (tid + j * NTHR) >> 3;
      const int t = u / NPIX;
      const int m = m0 + (u - t * NPIX);
      const bool inb = u < UNITS && m < p.M;
      const int ohw = p.OH * p.OW;
      const int ib = inb ? m / ohw : 0;
      const int r = m - ib * ohw;
      const int oh = inb ? r / p.OW : 0;
      const int ow = r - oh * p.OW;
      off16[j] = inb ? t * p.B + ib : -1;
      gpix[j] = ((oh * p.SH - p.PH) << 16) | ((ow * p.SW - p.PW) & 0xffff);
    }
  }
  auto load_pieces = [&](u32x4_t (&v)[PPT], int c) {
    if constexpr (KS == 0) {  // chunk c: tap c / nchunk, channels 64 (c % nchunk) ..
      const int tap = c / p.nchunk, cc = c - tap * p.nchunk;
      const int kh = tap / p.KW, kw = tap - kh * p.KW;
      const int piece = (tid & 7) * 16 + cc * 128;  // NTHR % 8 == 0: a thread's pieces share their index
#pragma unroll
      for (int j = 0; j < PPT; ++j) {
        const int ih = (gpix[j] >> 16) + kh * p.DH, iw = (int)(int16_t)(gpix[j] & 0xffff) + kw * p.DW;
        const bool inb = off16[j] >= 0 && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W;
        v[j] = inb ? *reinterpret_cast<const u32x4_t*>(p.in + ((off16[j] * p.H + ih) * p.W + iw) * (p.C * 2) + piece)
                   : u32x4_t{0u, 0u, 0u, 0u};
      }
    } else {
#pragma unroll
      for (int j = 0; j < PPT; ++j)
        v[j] = off16[j] >= 0 ? *reinterpret_cast<const u32x4_t*>(p.in + off16[j] + c * 128)
                             : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto store_pieces = [&](int buf, const u32x4_t (&v)[PPT]) {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int pc = tid + j * NTHR;
      if ((j + 1) * NTHR <= UNITS * 8 || pc < UNITS * 8) {
        const int u = pc >> 3, i = pc & 7;
        const int t = u / NPIX;
        const int e = t * TS + (u - t * NPIX) + (i >> 1) * NPIX + (i & 1) * (8 * NPIX + PAD);
        sB[buf][e] = uint2{v[j][0], v[j][1]};
        sB[buf][e + 4 * NPIX] = uint2{v[j][2], v[j][3]};
      }
    }
  };
  auto store_units = [&](int buf, const uint2 (&v)[UPT]) {
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
      if ((j + 1) * NTHR <= UNITS || tid + j * NTHR < UNITS) {
        u32x4_t pc[8];
        expand_word64(v[j], pc);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          // half-piece i, and 8 + i (the piece's other half) 4*NPIX entries on
          const int q = (i >> 1) * NPIX + (i & 1) * (8 * NPIX + PAD);
          sB[buf][soff[j] + q] = uint2{pc[i][0], pc[i][1]};
          sB[buf][soff[j] + q + 4 * NPIX] = uint2{pc[i][2], pc[i][3]};
        }
      }
    }
  };

  // ---- compute identity: this lane's B column / accumulator column
  int bbase, m;
  bool valid;
  if (KS == 3) {
    const int rb = wave / Gm::NCP;
    const int r_in = col >> 1;
    const int pr_ = rb * GR + r_in;
    const int pc0 = (wave - rb * Gm::NCP) * 2 + (col & 1);
    const bool pin = r_in < GR && pr_ < TR && pc0 < TC;
    // a lane outside the tile reads the pixels of a lane inside it (row rb*GR, its column)
    const int pr = pin ? pr_ : rb * GR;
    const int pc = pin ? pc0 : (pc0 < TC ? pc0 : 0);
    const int oh = oh0 + pr, ow = ow0 + pc;
    valid = pin && oh < p.OH && ow < p.OW;
    bbase = (g >> 1) * NPIX + (g & 1) * (8 * NPIX + PAD) + pr * Gm::HC + pc;  // half-piece g, halo pixel (pr, pc)
    m = valid ? (b * p.OH + oh) * p.OW + ow : 0;
  } else {
    const int pos = wave * 16 + col;
    valid = m0 + pos < p.M;
    bbase = (g >> 1) * NPIX + (g & 1) * (8 * NPIX + PAD) + pos;
    m = valid ? m0 + pos : 0;
  }

  // LDS byte address of this lane's tap-(0,0) half-piece g (half 0) in buffer 0; the four
  // 8-byte reads of a fragment are at compile-time offsets from it.
  const uint32_t lds0 =
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint2*)&sB[set * NBUF][0] + (uint32_t)bbase * 8u;
  // A operands through buffer resources: the (chunk, tap, group) offset is wave-uniform and
  // goes in the scalar offset, this lane's byte offset is one fixed VGPR and the tile index
  // an immediate, so a load costs no vector address arithmetic.
  const size_t wgroup = (size_t)p.nq * 4 * 64;
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<u32x4_t*>(p.wvals + (size_t)G0 * wgroup), 0, (int)(GPW * wgroup * sizeof(u32x4_t)), kBufferDword3);
  const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(p.wmeta + (size_t)G0 * wgroup), 0, (int)(GPW * wgroup * sizeof(uint32_t)), kBufferDword3);
  const int lv = lane * (int)sizeof(u32x4_t), lm = lane * 16;
  auto load_a = [&](int c, int tap, u32x4_t (&av)[GPW][4], uint32_t (&ix)[GPW][4]) {
    const int q = (tap * p.nchunk + c) * 4 * 64;
#pragma unroll
    for (int gg = 0; gg < GPW; ++gg)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int e = gg * (int)wgroup + q;  // entry offset, uniform
        av[gg][a] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rv, lv + a * 64 * (int)sizeof(u32x4_t),
                                                           e * (int)sizeof(u32x4_t), 0));
      }
#pragma unroll
    for (int gg = 0; gg < GPW; ++gg) {  // the lane's four tiles' metadata: one 16-byte load
      const u32x4_t m4 =
          __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rm, lm, (gg * (int)wgroup + q) * 4, 0));
#pragma unroll
      for (int a = 0; a < 4; ++a) ix[gg][a] = m4[a];
    }
  };

  float4_t acc[GPW][T][4];
#pragma unroll
  for (int gg = 0; gg < GPW; ++gg)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int a = 0; a < 4; ++a) acc[gg][t][a] = float4_t{0.f, 0.f, 0.f, 0.f};

  // the first A operands go out before the first staging loads: their latencies overlap
  u32x4_t av[NA][GPW][4];
  uint32_t ix[NA][GPW][4];
#pragma unroll
  for (int i = 0; i < PF; ++i) load_a(set, i, av[i], ix[i]);
  // Spike bits: the words of this set's next NQ chunks wait in registers, stq[i] holding chunk
  // c + (i + 1)*KSP while chunk c is reduced; they are loaded before the first barrier (all of
  // them for reductions of at most NQ + 1 chunks per set), not at the start of each chunk:
  // vector memory counts complete in issue order, so the wait for an A operand issued after a
  // staging load would also wait for that load, one or two taps later.
  constexpr int NQ = (PF == 2 || KSP == 2) ? 3 : 1;
  uint2 stq[NQ][UPT];
  u32x4_t pnext[IN_ENC == SENGINE_ENC_F16 ? PPT : 1];  // fp16 input: the next chunk's pieces
  if (IN_ENC == SENGINE_ENC_F16) {
    u32x4_t pcs[PPT];
    load_pieces(pcs, set);
    store_pieces(set * NBUF, pcs);
  } else {
    uint2 stg[UPT];
    load_units(stg, set);
#pragma unroll
    for (int i = 0; i < NQ; ++i)
      if (set + (i + 1) * KSP < p.nchunk) load_units(stq[i], set + (i + 1) * KSP);
    store_units(set * NBUF, stg);
  }
  __syncthreads();
  const int nloop = KS == 0 ? p.nq : p.nchunk;  // KS == 0: every chunk of every tap
  for (int c = set; c < nloop; c += KSP) {  // host: nloop % KSP == 0 (sets stay in step)
    const bool more = c + KSP < nloop;
    const int buf = NBUF == 2 ? ((c / KSP) & 1) : 0;
    if (IN_ENC == SENGINE_ENC_F16 && more) load_pieces(pnext, c + KSP);
    // B fragments: four ds_read_b64 per (tap, t), issued PF steps ahead of their SMFMACs
    // and waited for with an explicit lgkmcnt (the loop issues no other LDS operation).
    // Written as asm so the compiler neither fuses them into 16-byte or paired reads nor
    // hoists them further (both measured slower / register-starved).
    const uint32_t lbase = lds0 + (uint32_t)buf * (uint32_t)(BUFE * 8);  // within this set's buffers
    constexpr int NSTEP = NTAP * T;
    uint2 fr[NB][4];
    auto issue = [&](int step, uint2 (&f)[4]) {
      const int tp = step / T, t = step - (step / T) * T;
      const int toff = KS == 3 ? (tp / 3) * Gm::HC + (tp % 3) : 0;
      const int o = (t * TS + toff) * 8;
      // half-pieces g, 8 + g, 4 + g, 12 + g: +0, +4, +2, +6 NPIX from this lane's base
      asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(f[0]) : "v"(lbase), "i"(o));
      asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(f[1]) : "v"(lbase), "i"(o + 4 * NPIX * 8));
      asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(f[2]) : "v"(lbase), "i"(o + 2 * NPIX * 8));
      asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(f[3]) : "v"(lbase), "i"(o + 6 * NPIX * 8));
    };
#pragma unroll
    for (int i = 0; i < PF; ++i) issue(i, fr[i]);
#pragma unroll
    for (int tap = 0; tap < NTAP; ++tap) {
      // A operands PF taps ahead (crossing into the next chunk: they do not depend on LDS)
      const int ra = PF == 1 ? 0 : tap % NA;            // ring slot in use (PF = 2)
      const int rn = PF == 1 ? 1 : (tap + PF) % NA;     // ring slot being filled
      // PF = 2: unconditional (after the last chunk: this chunk's operands again, unused), so
      // the compiler's wait counts at the last taps need not merge a path with fewer loads in
      // flight; PF = 1 copies them into place at the end of the same tap (a wait for them), so
      // the last chunk skips them (one-chunk layers reach their epilogue without that wait)
      if (tap + PF < NTAP) load_a(c, tap + PF, av[rn], ix[rn]);
      else if (PF == 2 || more) load_a(more ? c + KSP : c, tap + PF - NTAP, av[rn], ix[rn]);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int step = tap * T + t;
        uint2(&f)[4] = fr[step % NB];
        // The wait names the fragment registers as operands, so every use of them is
        // ordered after it.
        if (step + PF < NSTEP) {
          issue(step + PF, fr[(step + PF) % NB]);
          if (PF == 2)
            asm volatile("s_waitcnt lgkmcnt(8)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]) :: "memory");
          else
            asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]) :: "memory");
        } else if (PF == 2 && step + 1 < NSTEP) {
          asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]) :: "memory");
        } else {
          asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]) :: "memory");
        }
        const half16_t bf = __builtin_bit_cast(
            half16_t, u32x8_t{f[0].x, f[0].y, f[1].x, f[1].y, f[2].x, f[2].y, f[3].x, f[3].y});
#pragma unroll
        for (int gg = 0; gg < GPW; ++gg)
#pragma unroll
          for (int a = 0; a < 4; ++a)
            acc[gg][t][a] = __builtin_amdgcn_smfmac_f32_16x16x64_f16(__builtin_bit_cast(half8_t, av[ra][gg][a]), bf,
                                                                     acc[gg][t][a], (int)ix[ra][gg][a], 0, 0);
      }
      if (PF == 1 && (tap + 1 < NTAP || more)) {
#pragma unroll
        for (int gg = 0; gg < GPW; ++gg)
#pragma unroll
          for (int a = 0; a < 4; ++a) {
            av[0][gg][a] = av[1][gg][a];
            ix[0][gg][a] = ix[1][gg][a];
          }
      }
    }
    if (more) {
      if (NBUF == 1) __syncthreads();  // every wave is done reading the single buffer
      if (IN_ENC == SENGINE_ENC_F16) {
        store_pieces(set * NBUF + (NBUF == 2 ? (buf ^ 1) : 0), pnext);
      } else {
        store_units(set * NBUF + (NBUF == 2 ? (buf ^ 1) : 0), stq[0]);
#pragma unroll
        for (int i = 0; i + 1 < NQ; ++i)
#pragma unroll
          for (int j = 0; j < UPT; ++j) stq[i][j] = stq[i + 1][j];
        // unconditional (clamped to this set's last chunk, then unused): no merged wait counts
        load_units(stq[NQ - 1], std::min(c + (NQ + 1) * KSP, p.nchunk - KSP + set));
      }
      __syncthreads();
    }
  }

  if (KSP == 2) {  // set 1's accumulators join set 0's through the (now free) LDS buffers
    static_assert(KSP == 1 || sizeof(sB) >= (size_t)NTHR * GPW * T * 4 * sizeof(float4_t), "LDS too small");
    float4_t* red = reinterpret_cast<float4_t*>(&sB[0][0]);
    __syncthreads();
    if (set == 1) {
#pragma unroll
      for (int gg = 0; gg < GPW; ++gg)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int a = 0; a < 4; ++a) red[((gg * T + t) * 4 + a) * NTHR + tid] = acc[gg][t][a];
    }
    __syncthreads();
    if (set == 1) return;
#pragma unroll
    for (int gg = 0; gg < GPW; ++gg)
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int a = 0; a < 4; ++a) acc[gg][t][a] += red[((gg * T + t) * 4 + a) * NTHR + tid];
  }

#pragma unroll
  for (int gg = 0; gg < GPW; ++gg) {
    const int cl = gg * 64 + g * 16;  // this lane's 16 channels within the block
    const EpiCoeffs cf{&sCoef[0][cl], &sCoef[1][cl], &sCoef[2][cl], &sCoef[3][cl]};
    lif_epilogue<T, OUT_ENC, MODE>(acc[gg], valid, m, p.M, p.F, G0 * 64 + cl, p.np, cf, p.state, p.out, p.h_trace,
                                   p.x_trace, p.sew);
  }
}

// Host side (fused_tile_host.hip).
struct TileShape {
  int KS, TR, TC, GR;
};

// fp16-input instances: T = 4, one channel group per wave (the reference ABI's fp16
// activations), bit or fp16 output, every epilogue mode; KSP = 2 (3x3, an even chunk count)
// splits the reduction over two wave sets for grids of at most one workgroup per CU.
template <int KS, int TR, int TC, int GR, int PF = 1, int KSP = 1>
hipError_t launch_tile_f16in(const TileParams& p, int out_enc, int mode, hipStream_t s) {
  constexpr int NTHR = TileGeom<KS, TR, TC, GR>::NTHR * KSP;
  const dim3 grid((unsigned)(p.ntiles * (p.F / 64)));
  constexpr int F16 = SENGINE_ENC_F16;
#define SENGINE_TILE_F16(OE, MODE_)                                                                                 \
  hipLaunchKernelGGL((fused_tile_kernel<4, KS, TR, TC, GR, 1, OE, MODE_, KSP, PF, F16>), grid, dim3(NTHR), 0, s, p)
  if (out_enc == SENGINE_ENC_BITS) {
    if (mode == EPI_LIF_HARD) SENGINE_TILE_F16(SENGINE_ENC_BITS, EPI_LIF_HARD);
    else if (mode == EPI_IF_HARD) SENGINE_TILE_F16(SENGINE_ENC_BITS, EPI_IF_HARD);
    else SENGINE_TILE_F16(SENGINE_ENC_BITS, EPI_GENERIC);
  } else {
    if (mode == EPI_LIF_HARD) SENGINE_TILE_F16(SENGINE_ENC_F16, EPI_LIF_HARD);
    else if (mode == EPI_IF_HARD) SENGINE_TILE_F16(SENGINE_ENC_F16, EPI_IF_HARD);
    else SENGINE_TILE_F16(SENGINE_ENC_F16, EPI_GENERIC);
  }
#undef SENGINE_TILE_F16
  return hipGetLastError();
}

template <int T, int KS, int TR, int TC, int GR, int GPW, int KSP = 1, int PF = 1>
hipError_t launch_tile(const TileParams& p, int out_enc, int mode, hipStream_t s) {
  constexpr int NTHR = TileGeom<KS, TR, TC, GR>::NTHR * KSP;
  const dim3 grid((unsigned)(p.ntiles * (p.F / (64 * GPW))));
  if (out_enc == SENGINE_ENC_BITS) {
    if (mode == EPI_LIF_HARD)
      hipLaunchKernelGGL((fused_tile_kernel<T, KS, TR, TC, GR, GPW, SENGINE_ENC_BITS, EPI_LIF_HARD, KSP, PF>), grid,
                         dim3(NTHR), 0, s, p);
    else if (mode == EPI_IF_HARD)
      hipLaunchKernelGGL((fused_tile_kernel<T, KS, TR, TC, GR, GPW, SENGINE_ENC_BITS, EPI_IF_HARD, KSP, PF>), grid,
                         dim3(NTHR), 0, s, p);
    else if (T == 4 && GPW == 1 && KS == 3 && mode == EPI_SHORTCUT)
      hipLaunchKernelGGL((fused_tile_kernel<T, KS, TR, TC, GR, GPW, SENGINE_ENC_BITS,
                                            (T == 4 && GPW == 1 && KS == 3) ? EPI_SHORTCUT : EPI_GENERIC, KSP, PF>),
                         grid, dim3(NTHR), 0, s, p);
    else
      hipLaunchKernelGGL((fused_tile_kernel<T, KS, TR, TC, GR, GPW, SENGINE_ENC_BITS, EPI_GENERIC, KSP, PF>), grid,
                         dim3(NTHR), 0, s, p);
  } else if ((KS == 1 || KS == 3) && T == 4 && mode == EPI_LIF_HARD) {
    // fp16 output (token Linears and a transformer stem's last conv writing the fp16 residual
    // stream): fast epilogue
    hipLaunchKernelGGL((fused_tile_kernel<T, KS, TR, TC, GR, GPW, SENGINE_ENC_F16,
                                          ((KS == 1 || KS == 3) && T == 4) ? EPI_LIF_HARD : EPI_GENERIC, KSP, PF>),
                       grid, dim3(NTHR), 0, s, p);
  } else {
    hipLaunchKernelGGL((fused_tile_kernel<T, KS, TR, TC, GR, GPW, SENGINE_ENC_F16, EPI_GENERIC, KSP, PF>), grid,
                       dim3(NTHR), 0, s, p);
  }
  return hipGetLastError();
}

// Launchers compiled in fused_tile3.hip (KS = 3) and fused_tile1.hip (KS = 1).  ksplit: 1
// or 2 (3x3, T = 4, one channel group per wave, nchunk even).
hipError_t launch_tile3(const TileParams& p, int T, int shape, int gpw, int ksplit, int pf, int out_enc, int mode,
                        hipStream_t s);
hipError_t launch_tile1(const TileParams& p, int T, int gpw, int out_enc, int mode, hipStream_t s);
// fp16 input (T = 4): the 3x3 tile shapes (fused_tile3.hip; ksplit 1 or 2), the 1x1 tile kernel
// (fused_tile1.hip)
hipError_t launch_tile3_f16in(const TileParams& p, int shape, int ksplit, int out_enc, int mode, hipStream_t s);
// The persistent 3x3 form (tile3ps.h) of a tile shape, on `slots` resident workgroups.
hipError_t launch_tile3_persistent(const TileParams& p, int shape, int mode, int slots, hipStream_t s);
// ... its paired-tail form (the blob of compress_2_4_tail; p.nq its chunk count).
hipError_t launch_tile3_persistent_pair(const TileParams& p, int shape, int mode, int slots, hipStream_t s);

}  // namespace sengine
