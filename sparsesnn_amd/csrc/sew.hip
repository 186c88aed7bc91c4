// The layers of a SEW-ResNet around the fused Conv+BN+LIF op (models/sewresnet.py:123-210):
// the dense stem convolution on image pixels, the neuron over the stem output repeated over
// T, max-pooling of spike bits, and the pooled / time-averaged Linear head.  All of them
// are small next to the fused convolutions; they are HBM- or launch-bound.
#include "common.h"
#include "internal.h"

namespace sengine {

// ---- stem: dense fp32 convolution (any kernel / stride / pad) + folded BN ----------------
// x: NCHW fp32 images (N, C_in, H, W) (the reference feeds the raw 4-D batch to conv1,
// models/sewresnet.py:199); w: OIHW or HWIO fp32; out: NHWC fp32 (N, OH, OW, C_out);
// accumulation in (c_in, kh, kw) order in fp32 like the reference's CPU conv.
// Fast path (HWIO, C_out % 16 == 0, the input rows of 256 output pixels fit in LDS): each
// thread computes 8 or 16 output channels of one pixel from LDS-staged input, with the
// weights in SGPRs.  Generic path: one output value per thread.  The stem + neuron entry runs
// 3-channel 7x7 / 3x3 stems of 32 or 64 channels on the fp32 matrix cores instead
// (stem_mfma_kernel), summing the taps in a different order.
struct StemParams {
  const float* x;
  const float* w;
  const float* scale;
  const float* bias;
  float* out;
  int N, C, H, W, F, KH, KW, SH, SW, PH, PW, OH, OW;
  // fused neuron (+ max-pool): stem_conv_bn_lds_kernel<KW, kStemPool / kStemSpikes, CPT>
  uint16_t* spikes;  // (T, N, OH, OW) x F bits, or null
  uint16_t* pooled;  // (T, N, POH, POW) x F bits
  int T, PK, PS, PP, POH, POW;
  NeuronParams np;
};

constexpr int kStemPix = 256;        // output pixels (of one image) per workgroup
constexpr int kStemLdsInput = 12288; // staged, zero-padded input floats (at most)
constexpr int kStemMaxT = 16;        // fused variant: spike words of all T kept in LDS for the pool
constexpr int kStemRows = 6;         // row-wise staging: rows per wave whose loads are in flight together
constexpr int kStemFlat = 16;        // flat staging: floats in flight per thread of a 256-thread workgroup
constexpr int kStemTouchTaps = 160;  // weight taps (64-byte lines) prefetched into the scalar cache

// Exact n / d for 0 <= n < 2^16 and 1 <= d < 2^16 by a multiply-high with m = ceil(2^32 / d):
// with e = m*d - 2^32 < d, n*m / 2^32 = n/d + n*e / (d * 2^32) and n*e < 2^32, so the
// fraction added never carries past the next integer.
struct StemDiv {
  uint32_t m, d;
  __device__ explicit StemDiv(uint32_t d_) : m(d_ > 1 ? (uint32_t)(0xffffffffull / d_ + 1) : 0u), d(d_) {}
  __device__ uint32_t operator()(uint32_t n) const { return d > 1 ? __umulhi(n, m) : n; }
};

typedef const float4_t __attribute__((address_space(4)))* StemWPtr;

// Brings the scalar-cache lines at base + off[i] bytes (wave-uniform) in: eight scalar loads
// issued back to back, then one wait, so the eight misses overlap.  Loads only; the loaded
// words are discarded.  The outputs are early-clobber: a load may land while later loads of
// the block still read their base and offset registers.
__device__ inline void stem_touch8(const float* base, const int (&off)[8]) {
  uint32_t d0, d1, d2, d3, d4, d5, d6, d7;
  asm volatile(
      "s_load_dword %0, %8, %9\n\t"
      "s_load_dword %1, %8, %10\n\t"
      "s_load_dword %2, %8, %11\n\t"
      "s_load_dword %3, %8, %12\n\t"
      "s_load_dword %4, %8, %13\n\t"
      "s_load_dword %5, %8, %14\n\t"
      "s_load_dword %6, %8, %15\n\t"
      "s_load_dword %7, %8, %16\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(d0), "=&s"(d1), "=&s"(d2), "=&s"(d3), "=&s"(d4), "=&s"(d5), "=&s"(d6), "=&s"(d7)
      : "s"(base), "s"(off[0]), "s"(off[1]), "s"(off[2]), "s"(off[3]), "s"(off[4]), "s"(off[5]), "s"(off[6]),
        "s"(off[7]));
}

// Stages the C x nrows input rows (from ih0) of image xn into sx, zero-padded by PW columns on
// each side (row c * nrows + r, then column; WP = W + 2 * PW) with the NT threads of a
// workgroup.  Rows of at least 128 floats: wave w copies staged rows w, w + NW, ..., lane l
// columns l, l + 64, ..., the loads of kStemRows rows x 4 column chunks issued before any of
// them is stored; narrow rows: thread i copies staged floats i, i + NT, ..., FLAT loads in flight.
template <int NT>
__device__ __forceinline__ void stem_stage_rows(const StemParams& p, float* sx, const float* xn, int ih0, int nrows,
                                                int WP) {
  constexpr int NW = NT / 64;
  constexpr int FLAT = kStemFlat * 256 / NT;
  const int nrow_st = p.C * nrows;
  const int nx = nrow_st * WP;
  if (WP >= 128) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    for (int col0 = 0; col0 < WP; col0 += 4 * 64)
      for (int row0 = wave; row0 < nrow_st; row0 += NW * kStemRows) {
        float v[kStemRows][4];
#pragma unroll
        for (int u = 0; u < kStemRows; ++u) {
          const int row = row0 + NW * u;
          const int c = row / nrows;
          const int ih = ih0 + row - c * nrows;
          const bool row_ok = row < nrow_st && ih >= 0 && ih < p.H;
          const float* xr = xn + ((int64_t)c * p.H + ih) * p.W;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int iw = col0 + 64 * j + lane - p.PW;
            v[u][j] = row_ok && iw >= 0 && iw < p.W ? xr[iw] : 0.f;
          }
        }
#pragma unroll
        for (int u = 0; u < kStemRows; ++u) {
          const int row = row0 + NW * u;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int col = col0 + 64 * j + lane;
            if (row < nrow_st && col < WP) sx[row * WP + col] = v[u][j];
          }
        }
      }
  } else {
    const StemDiv by_wp(WP), by_rows(nrows);
    for (int i0 = threadIdx.x; i0 < nx; i0 += FLAT * NT) {
      float v[FLAT];
#pragma unroll
      for (int u = 0; u < FLAT; ++u) {
        const int i = i0 + u * NT;
        const int row = (int)by_wp((uint32_t)i);
        const int c = (int)by_rows((uint32_t)row);
        const int ih = ih0 + row - c * nrows;
        const int iw = i - row * WP - p.PW;
        v[u] = i < nx && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W ? xn[((int64_t)c * p.H + ih) * p.W + iw] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < FLAT; ++u)
        if (i0 + u * NT < nx) sx[i0 + u * NT] = v[u];
    }
  }
}

// Workgroup = (image n, block of kStemPix output pixels in (oh, ow) order, 16-channel group
// fg); thread = one output pixel x CPT channels (CPT = 8: two threads per pixel, waves
// 0-3 channels 0-7 of the group and waves 4-7 channels 8-15, so a small grid still has two
// waves per SIMD).  The workgroup stages the input rows the block reads, with the padding
// as zeros, in dynamic LDS sized to the block; the tap loop then has no bounds checks.  The
// weights of a wave's channels are the same for all its lanes, so they are read from global
// memory at wave-uniform addresses (constant address space: scalar loads into SGPRs, which
// the FMAs take as operands) -- read from LDS, every 16 FMAs would need a 1 KB wave-wide
// float4 broadcast read, which kept the tap loop LDS-bound.
// What the LDS stem kernel does after the convolution.
enum StemMode : int {
  kStemOut = 0,    // folded BN -> fp32 NHWC out
  kStemPool = 1,   // folded BN -> neuron over T repeats -> spike max-pool (whole image per workgroup)
  kStemSpikes = 2  // folded BN -> fp32 out (if p.out) and neuron over T repeats -> spike bits
};

template <int KW_, int MODE, int CPT>
__global__ __launch_bounds__(kStemPix * 16 / CPT) void stem_conv_bn_lds_kernel(StemParams p) {
  static_assert(CPT == 16 || CPT == 8, "8 or 16 channels per thread");
  constexpr int NT = kStemPix * 16 / CPT;
  constexpr int NW = NT / 64;
  extern __shared__ float sx[];  // staged input (row = c * nrows + r, then column); fused: spike words after it
  const int KW = KW_ > 0 ? KW_ : p.KW;
  const int fgroups = p.F / 16;
  const int pblocks = (p.OH * p.OW + kStemPix - 1) / kStemPix;
  const int fg = blockIdx.x % fgroups;
  const int pb = (blockIdx.x / fgroups) % pblocks;
  const int n = blockIdx.x / (fgroups * pblocks);
  const int pix0 = pb * kStemPix;
  const int oh_first = pix0 / p.OW;
  const int oh_last = min(p.OH - 1, (pix0 + kStemPix - 1) / p.OW);
  const int ih0 = oh_first * p.SH - p.PH;
  const int nrows = (oh_last - oh_first) * p.SH + p.KH;
  const int WP = p.W + 2 * p.PW;  // padded row
  const int nx = p.C * nrows * WP;
  const float* xn = p.x + (int64_t)n * p.C * p.H * p.W;
  // Weight prefetch: the tap loop's scalar loads come one (c, kh) row at a time, each row
  // waited for before its FMAs, so a workgroup that finds the scalar cache cold (small
  // grids: one workgroup per CU) would pay one L2/HBM round trip per row.  Wave w first
  // touches the 64-byte lines of taps w, w + NW, ... with scalar loads issued eight at a
  // time, one round trip per eight lines.
  {
    const int last = p.KH * KW * p.C - 1;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const float* wl = p.w + fg * 16;
#pragma unroll
    for (int i0 = 0; i0 < (kStemTouchTaps + NW - 1) / NW; i0 += 8) {
      int off[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) off[i] = min(wv + NW * (i0 + i), last) * p.F * (int)sizeof(float);
      stem_touch8(wl, off);
    }
  }
  stem_stage_rows<NT>(p, sx, xn, ih0, nrows, WP);
  __syncthreads();
  const int part = CPT == 16 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kStemPix));
  const int tpix = (int)(threadIdx.x % kStemPix);
  const int pix_ = pix0 + tpix;
  const bool valid = pix_ < p.OH * p.OW;
  if (MODE != kStemPool && !valid) return;
  const int pix = valid ? pix_ : pix0;  // the pooling variant keeps every thread for its barriers
  const int oh = pix / p.OW;
  const int ow = pix - oh * p.OW;
  const float* xb = &sx[(oh - oh_first) * p.SH * WP + ow * p.SW];
  float acc[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) acc[j] = 0.f;
  // HWIO weights: tap (kh, kw, c) of channel f at ((kh*KW + kw)*C + c)*F + f
  const int ch0 = fg * 16 + part * CPT;
  const StemWPtr wg = (StemWPtr)(p.w + ch0);
  const int wtap = p.F / 4;  // float4 stride between consecutive (kh, kw, c) taps
  for (int c = 0; c < p.C; ++c)
    for (int kh = 0; kh < p.KH; ++kh) {
      const float* xr = xb + (c * nrows + kh) * WP;
      const StemWPtr wr = wg + ((kh * KW) * p.C + c) * wtap;
      if (KW_ > 0) {
        float xv[KW_ > 0 ? KW_ : 1];
#pragma unroll
        for (int kw = 0; kw < (KW_ > 0 ? KW_ : 1); ++kw) xv[kw] = xr[kw];
#pragma unroll
        for (int kw = 0; kw < (KW_ > 0 ? KW_ : 1); ++kw) {
#pragma unroll
          for (int q = 0; q < CPT / 4; ++q) {
            const float4_t w1 = wr[kw * p.C * wtap + q];
            acc[4 * q + 0] = __builtin_fmaf(xv[kw], w1.x, acc[4 * q + 0]);
            acc[4 * q + 1] = __builtin_fmaf(xv[kw], w1.y, acc[4 * q + 1]);
            acc[4 * q + 2] = __builtin_fmaf(xv[kw], w1.z, acc[4 * q + 2]);
            acc[4 * q + 3] = __builtin_fmaf(xv[kw], w1.w, acc[4 * q + 3]);
          }
        }
      } else {
        for (int kw = 0; kw < KW; ++kw) {
          const float x1 = xr[kw];
#pragma unroll
          for (int q = 0; q < CPT / 4; ++q) {
            const float4_t w1 = wr[kw * p.C * wtap + q];
            acc[4 * q + 0] = __builtin_fmaf(x1, w1.x, acc[4 * q + 0]);
            acc[4 * q + 1] = __builtin_fmaf(x1, w1.y, acc[4 * q + 1]);
            acc[4 * q + 2] = __builtin_fmaf(x1, w1.z, acc[4 * q + 2]);
            acc[4 * q + 3] = __builtin_fmaf(x1, w1.w, acc[4 * q + 3]);
          }
        }
      }
    }
  const float* sc = p.scale + ch0;
  const float* bi = p.bias + ch0;
  if (MODE == kStemOut) {
    float* o = p.out + (((int64_t)n * p.OH + oh) * p.OW + ow) * p.F + ch0;
#pragma unroll
    for (int j = 0; j < CPT; j += 4)
      *reinterpret_cast<float4*>(o + j) =
          float4{__builtin_fmaf(acc[j], sc[j], bi[j]), __builtin_fmaf(acc[j + 1], sc[j + 1], bi[j + 1]),
                 __builtin_fmaf(acc[j + 2], sc[j + 2], bi[j + 2]), __builtin_fmaf(acc[j + 3], sc[j + 3], bi[j + 3])};
    return;
  }
  if (MODE == kStemSpikes) {
    // The stem output (stored as by kStemOut when p.out is set) and the neuron over it
    // repeated T times with the arithmetic of repeat_neuron_kernel; the CPT spike bits of
    // (t, pixel) form 16-bit word fg of the pixel's F/16 words.
    float xo[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) xo[j] = __builtin_fmaf(acc[j], sc[j], bi[j]);
    const int64_t opix = ((int64_t)n * p.OH + oh) * p.OW + ow;
    if (p.out) {
      float* o = p.out + opix * p.F + ch0;
#pragma unroll
      for (int j = 0; j < CPT; j += 4)
        *reinterpret_cast<float4*>(o + j) = float4{xo[j], xo[j + 1], xo[j + 2], xo[j + 3]};
    }
    float v[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      if (p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2) xo[j] *= p.np.rtau;  // exact
      v[j] = 0.f;
    }
    const int64_t tstride = (int64_t)p.N * p.OH * p.OW * (p.F / 16);
    uint16_t* so = p.spikes + opix * (p.F / 16) + ch0 / 16;
    for (int t = 0; t < p.T; ++t) {
      uint32_t word = 0;
#pragma unroll
      for (int j = 0; j < CPT; ++j) {
        const float h = neuron_charge(p.np, v[j], xo[j]);
        const bool spike = h >= p.np.vth;
        v[j] = neuron_reset(p.np, h, spike);
        word |= (uint32_t)spike << j;
      }
      so[t * tstride] = (uint16_t)word;
    }
    return;
  }
  // The neuron on the stem output repeated over T (models/sewresnet.py:201-202), the same
  // arithmetic as repeat_neuron_kernel: CPT spike bits per t for this pixel, into the
  // 16-bit word of (t, pixel) after the staged input (bits 0-7 from part 0, 8-15 from part 1).
  uint16_t* sspk = reinterpret_cast<uint16_t*>(sx + ((nx + 3) & ~3));
  float xf[CPT], v[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const float x = __builtin_fmaf(acc[j], sc[j], bi[j]);
    xf[j] = (p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2) ? x * p.np.rtau : x;  // exact
    v[j] = 0.f;
  }
  __syncthreads();  // every thread is done reading the staged input before spikes land next to it
  for (int t = 0; t < p.T; ++t) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const float h = neuron_charge(p.np, v[j], xf[j]);
      const bool spike = h >= p.np.vth;
      v[j] = neuron_reset(p.np, h, spike);
      word |= (uint32_t)spike << j;
    }
    if (CPT == 16)
      sspk[t * kStemPix + tpix] = (uint16_t)word;
    else
      reinterpret_cast<uint8_t*>(sspk)[(t * kStemPix + tpix) * 2 + part] = (uint8_t)word;
  }
  __syncthreads();
  const int npix = p.OH * p.OW;
  const int fw = p.F / 16;  // 16-bit spike words per pixel
  if (p.spikes)
    for (int i = threadIdx.x; i < p.T * npix; i += NT) {
      const int t = i / npix;
      const int q = i - t * npix;
      p.spikes[((int64_t)(t * p.N + n) * npix + q) * fw + fg] = sspk[t * kStemPix + q];
    }
  // max-pool of the spikes (models/sewresnet.py:143,203): OR over the in-image taps
  const int npool = p.POH * p.POW;
  for (int i = threadIdx.x; i < p.T * npool; i += NT) {
    const int t = i / npool;
    const int q = i - t * npool;
    const int ph = q / p.POW;
    const int pw = q - ph * p.POW;
    uint32_t m = 0;
    for (int kh = 0; kh < p.PK; ++kh) {
      const int ih = ph * p.PS - p.PP + kh;
      if (ih < 0 || ih >= p.OH) continue;
      for (int kw = 0; kw < p.PK; ++kw) {
        const int iw = pw * p.PS - p.PP + kw;
        if (iw >= 0 && iw < p.OW) m |= sspk[t * kStemPix + ih * p.OW + iw];
      }
    }
    p.pooled[((int64_t)(t * p.N + n) * npool + q) * fw + fg] = (uint16_t)m;
  }
}

// Stem + neuron on the fp32 matrix cores (v_mfma_f32_16x16x4_f32, 4 taps per instruction):
// the convolution as a GEMM of (output pixels) x (C_ * KH_ * KW_ taps, HWIO order: tap k =
// (kh * KW + kw) * C + c, zero weights past the last tap) x (channels).  Workgroup = (image n,
// 16 NB output pixels), NWV waves, wave w = channels 16w..16w+15 of all of them (NB 16-pixel
// blocks, 4 NB accumulators per lane); the staged input rows are read by all waves.
// Lane l supplies, per 4-tap step s, the input value of pixel l % 16 of each block at tap
// 4s + l / 16 (the taps' staged-input offsets in an LDS table, its weights in registers) and
// its weight for channel l % 16; it ends holding pixels 4 (l / 16) + r, r < 4, of each block for that channel.
// Epilogue as in stem_conv_bn_lds_kernel<..., kStemSpikes, ...> (same BN, neuron arithmetic
// and output layouts); a wave's 16-channel spike word of a pixel is the ballot of its spike
// compare, picked out of the 64-lane mask by the lane that stores it.  The products are
// summed in a different order than the FMA kernels', so outputs agree to fp32 rounding.
// FASTN: hard-reset LIF with power-of-two 1/tau and 1 - 1/tau, or hard-reset IF, whose charge
// is one fma (IF: v * 1 + x, the same single rounding as v + x); else the generic neuron.
template <int C_, int KH_, int KW_, int NWV, bool FASTN, int NB>
__global__ __launch_bounds__(64 * NWV) void stem_mfma_kernel(StemParams p) {
  constexpr int NT = 64 * NWV;
  constexpr int K = C_ * KH_ * KW_;
  constexpr int KS = (K + 3) / 4;
  constexpr int PIX = 16 * NB;  // output pixels per workgroup
  // LDS: the staged-input offsets of the 4 KS taps (int), then the staged input rows
  extern __shared__ float lds_stem[];
  int* const sk = reinterpret_cast<int*>(lds_stem);
  float* const sx = lds_stem + 4 * KS;
  const int npix = p.OH * p.OW;
  const int pblocks = (npix + PIX - 1) / PIX;
  const int pb = blockIdx.x % pblocks;
  const int n = blockIdx.x / pblocks;
  const int pix0 = pb * PIX;
  const int oh_first = pix0 / p.OW;
  const int oh_last = min(p.OH - 1, (pix0 + PIX - 1) / p.OW);
  const int ih0 = oh_first * p.SH - p.PH;
  const int nrows = (oh_last - oh_first) * p.SH + KH_;
  const int WP = p.W + 2 * p.PW;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int q = lane >> 4, j = lane & 15;
  const int ch = wv * 16 + j;
  float wb[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int k = 4 * s + q;
    wb[s] = k < K ? p.w[(int64_t)k * p.F + ch] : 0.f;
  }
  for (int k = threadIdx.x; k < 4 * KS; k += NT) {
    const int kk = k < K ? k : K - 1;  // a real tap of the same pixel; its weight is zero
    const int c = kk % C_, khw = kk / C_;
    sk[k] = (c * nrows + khw / KW_) * WP + khw % KW_;
  }
  stem_stage_rows<NT>(p, sx, p.x + (int64_t)n * C_ * p.H * p.W, ih0, nrows, WP);
  __syncthreads();
  // Pixel pix0 + 16 b + j of block b (past the image: pixel pix0, computed but not stored).
  // Every staged offset read is below C * nrows * WP: (OW - 1) * SW + KW - 1 < W + 2 * PW.
  int base[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int pix = min(pix0 + 16 * b + j, npix - 1);
    const int oh = pix / p.OW;
    base[b] = (oh - oh_first) * p.SH * WP + (pix - oh * p.OW) * p.SW;
  }
  float4_t acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int koff = sk[4 * s + q];
    float a[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) a[b] = sx[base[b] + koff];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[b], wb[s], acc[b], 0, 0, 0);
  }
  const float sc = p.scale[ch], bi = p.bias[ch];
  const bool fold = p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2;
  const float dec = p.np.neuron == SENGINE_NEURON_IF ? 1.f : p.np.decay;
  const int fw = p.F / 16;
  const int64_t tstride = (int64_t)p.N * npix * fw;
  // the word this lane stores (lanes 0-15): pixel 4 g + r of a block, g = j / 4, r = j % 4
  const int rsel = j & 3, gsh = 16 * (j >> 2);
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    float xo[4], v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      xo[r] = __builtin_fmaf(acc[b][r], sc, bi);
      const int pix = pix0 + 16 * b + 4 * q + r;
      if (p.out && pix < npix) p.out[((int64_t)n * npix + pix) * p.F + ch] = xo[r];
      if (fold) xo[r] *= p.np.rtau;  // exact
      v[r] = 0.f;
    }
    const int spix = pix0 + 16 * b + j;
    uint16_t* so = p.spikes + ((int64_t)n * npix + spix) * fw + wv;
    const bool st = q == 0 && spix < npix;
    for (int t = 0; t < p.T; ++t) {
      uint64_t mk[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float h = FASTN ? __builtin_fmaf(v[r], dec, xo[r]) : neuron_charge(p.np, v[r], xo[r]);
        const bool spike = h >= p.np.vth;
        v[r] = FASTN ? (spike ? p.np.vreset : h) : neuron_reset(p.np, h, spike);
        mk[r] = __builtin_amdgcn_ballot_w64(spike);
      }
      const uint64_t m = rsel == 0 ? mk[0] : rsel == 1 ? mk[1] : rsel == 2 ? mk[2] : mk[3];
      if (st) so[t * tstride] = (uint16_t)(m >> gsh);
    }
  }
}

template <int HWIO>
__global__ __launch_bounds__(256) void stem_conv_bn_kernel(StemParams p) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.N * p.OH * p.OW * p.F;
  if (i >= total) return;
  const int f = (int)(i % p.F);
  int64_t r = i / p.F;
  const int ow = (int)(r % p.OW);
  r /= p.OW;
  const int oh = (int)(r % p.OH);
  const int n = (int)(r / p.OH);
  float acc = 0.f;
  for (int c = 0; c < p.C; ++c) {
    const float* xc = p.x + ((int64_t)n * p.C + c) * p.H * p.W;
    for (int kh = 0; kh < p.KH; ++kh) {
      const int ih = oh * p.SH - p.PH + kh;
      if (ih < 0 || ih >= p.H) continue;
      for (int kw = 0; kw < p.KW; ++kw) {
        const int iw = ow * p.SW - p.PW + kw;
        if (iw < 0 || iw >= p.W) continue;
        const float wv = HWIO ? p.w[(((int64_t)kh * p.KW + kw) * p.C + c) * p.F + f]
                              : p.w[(((int64_t)f * p.C + c) * p.KH + kh) * p.KW + kw];
        acc = __builtin_fmaf(xc[ih * p.W + iw], wv, acc);
      }
    }
  }
  p.out[i] = __builtin_fmaf(acc, p.scale[f], p.bias[f]);
}

// ---- neuron over an input repeated at every timestep (models/sewresnet.py:201-202) -------
struct RepeatNeuronParams {
  const float* x;  // n values, the same at every t
  uint32_t* out;   // spike bits (T, n)
  int64_t n;
  int T;
  NeuronParams np;
};

__global__ __launch_bounds__(256) void repeat_neuron_kernel(RepeatNeuronParams p) {
  const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool valid = s < p.n;
  const int lane = threadIdx.x & 63;
  const float x = valid ? p.x[s] : 0.f;
  float xf = x;
  if (p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2) xf = x * p.np.rtau;  // exact
  float v = 0.f;
  for (int t = 0; t < p.T; ++t) {
    const float h = neuron_charge(p.np, v, xf);
    const bool spike = valid && h >= p.np.vth;
    v = neuron_reset(p.np, h, spike);
    const uint64_t mask = __ballot(spike);
    // n % 32 == 0: a 32-lane half-wave is one output word when its first lane is valid
    if ((lane & 31) == 0 && valid) p.out[((int64_t)t * p.n + s) >> 5] = (uint32_t)(mask >> (lane & 32));
  }
}

// ---- max-pooling of spike bits: the max of {0,1} values is their OR ----------------------
// (SeqToANNContainer(MaxPool2d(k, s, p)), models/sewresnet.py:143,203; padding never wins a
// max, so out-of-image taps are skipped).  One thread per (image-timestep, oh, ow, 32-bit word).
struct PoolParams {
  const uint32_t* in;
  uint32_t* out;
  int NT, H, W, CW, K, S, P, OH, OW;  // CW: 32-bit words per pixel
};

__global__ __launch_bounds__(256) void maxpool_bits_kernel(PoolParams p) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.NT * p.OH * p.OW * p.CW;
  if (i >= total) return;
  const int cw = (int)(i % p.CW);
  int64_t r = i / p.CW;
  const int ow = (int)(r % p.OW);
  r /= p.OW;
  const int oh = (int)(r % p.OH);
  const int64_t nt = r / p.OH;
  uint32_t acc = 0;
  for (int kh = 0; kh < p.K; ++kh) {
    const int ih = oh * p.S - p.P + kh;
    if (ih < 0 || ih >= p.H) continue;
    for (int kw = 0; kw < p.K; ++kw) {
      const int iw = ow * p.S - p.P + kw;
      if (iw < 0 || iw >= p.W) continue;
      acc |= p.in[((nt * p.H + ih) * p.W + iw) * p.CW + cw];
    }
  }
  p.out[i] = acc;
}

// ---- head: global average pool per timestep, mean over T, Linear ------------------------
// (models/sewresnet.py:208-210; models/msresnet.py:155-160).  in: integer activations as
// `planes` bit planes, NHWC with planes*C channels, (T*B, HW) positions.  Workgroup (image,
// slice of the outputs): the per-channel sums are exact integers, counted once per
// workgroup -- thread (word column wi, position slice) walks its slice of the T*HW positions
// with coalesced word reads and counts in SWAR lanes and registers, then adds into LDS
// -- and scaled once into fp32 features; each wave then owns HEAD_OPW outputs at a time
// (looping over the workgroup's slice of the outputs), its lanes split the reduction over C
// (coalesced reads of the Linear weight rows) and a cross-lane sum finishes each output.
constexpr int HEAD_OPW = 4;        // outputs per wave and pass
constexpr int HEAD_MAX_PC = 8192;  // planes * C held as integer counters in LDS
struct HeadParams {
  const uint32_t* in;
  const float* w;  // (N_out, C) fp32, nn.Linear layout
  const float* b;  // (N_out)
  float* out;      // (B, N_out)
  int T, B, HW, C, planes, N_out;
  const int32_t* partial = nullptr;  // fp16 input split over workgroups: (B, nsplit, C) sums
  int nsplit = 0;
};

// Per-channel integer sums of an integer-valued fp16 stream (T*B, HW, C), split over
// `nsplit` workgroups per image: workgroup (s, b) sums positions q = t*HW + p in
// [s*P/nsplit, (s+1)*P/nsplit) of image b (P = T*HW; exact in int32) into
// partial[(b*nsplit + s)*C + c].  The head then adds the nsplit sums of a channel.  One
// workgroup per image had each CU stream an image's whole 16-bit stream alone.
__global__ __launch_bounds__(256) void token_sums_kernel(const _Float16* in, int T, int B, int HW, int C, int nsplit,
                                                         int32_t* partial) {
  __shared__ int cnt[HEAD_MAX_PC];
  const int s = blockIdx.x, b = blockIdx.y;
  for (int i = threadIdx.x; i < C; i += 256) cnt[i] = 0;
  __syncthreads();
  const int64_t P = (int64_t)T * HW;
  const int q0 = (int)(P * s / nsplit), q1 = (int)(P * (s + 1) / nsplit);
  const int per8 = C / 8;              // 16-byte column groups
  const int nsl = 256 / per8;          // position slices of the workgroup
  const int sl = (int)threadIdx.x / per8;
  const int c8 = ((int)threadIdx.x - sl * per8) * 8;
  if (sl < nsl) {
    int s8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int t = (q0 + sl) / HW, sp = q0 + sl - t * HW;
    for (int q = q0 + sl; q < q1; q += nsl) {
      const half8_t v = *reinterpret_cast<const half8_t*>(in + (((int64_t)t * B + b) * HW + sp) * C + c8);
#pragma unroll
      for (int e = 0; e < 8; ++e) s8[e] += (int)(float)v[e];
      sp += nsl;
      while (sp >= HW) {
        sp -= HW;
        ++t;
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (s8[e]) atomicAdd(&cnt[c8 + e], s8[e]);
  }
  __syncthreads();
  for (int c = threadIdx.x; c < C; c += 256) partial[((int64_t)b * nsplit + s) * C + c] = cnt[c];
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <int NT>
__global__ __launch_bounds__(NT) void sew_head_kernel(HeadParams p) {
  __shared__ int cnt[HEAD_MAX_PC];
  __shared__ float feat[HEAD_MAX_PC];
  const int bimg = blockIdx.x;
  const int fp16in = p.planes == 0;  // integer-valued fp16 stream instead of bit planes
  const int planes = fp16in ? 1 : p.planes;
  const int words = fp16in ? 0 : planes * p.C / 32;
  const int npos = p.T * p.HW;  // (t, s) positions of this image
  for (int i = threadIdx.x; i < planes * p.C; i += NT) cnt[i] = 0;
  __syncthreads();
  if (p.partial) {  // fp16 input summed by token_sums_kernel: add its nsplit partial sums
    for (int c = threadIdx.x; c < p.C; c += NT) {
      int sum = 0;
      for (int s = 0; s < p.nsplit; ++s) sum += p.partial[((int64_t)bimg * p.nsplit + s) * p.C + c];
      cnt[c] = sum;
    }
  } else if (fp16in) {
    // 8 channels (16 bytes) per thread and position, integer sums (exact) per channel
    const int per8 = p.C / 8;
    const int nsl = NT / per8;
    const int sl = (int)threadIdx.x / per8;
    const int c8 = ((int)threadIdx.x - sl * per8) * 8;
    if (sl < nsl) {
      int s8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      const _Float16* base = reinterpret_cast<const _Float16*>(p.in);
      for (int q = sl; q < npos; q += nsl) {
        const int t = q / p.HW;
        const int sp = q - t * p.HW;
        const half8_t v = *reinterpret_cast<const half8_t*>(base + (((int64_t)t * p.B + bimg) * p.HW + sp) * p.C + c8);
#pragma unroll
        for (int e = 0; e < 8; ++e) s8[e] += (int)(float)v[e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (s8[e]) atomicAdd(&cnt[c8 + e], s8[e]);
    }
  }
  const int per = words < NT ? (words > 0 ? words : 1) : NT;  // word columns per pass
  const int nslice = NT / per;
  const int slice = (int)threadIdx.x / per;
  // Bit counting in SWAR lanes: nibble n of a / b / c / d counts channel 4n / 4n+1 / 4n+2 /
  // 4n+3 of the word column (3 VALU per word and lane set, flushed every 15 words before a
  // nibble can overflow), their even / odd nibbles go into byte counters (flushed every
  // 17 x 15 = 255 words), and those into 32 integer counters: ~12 VALU per word instead of
  // two per bit; the last < 15 positions of a thread are added bit by bit.  Exact.
  for (int wbase = 0; wbase < words; wbase += per) {
    const int wi = wbase + (int)threadIdx.x % per;
    if (slice >= nslice || wi >= words) continue;
    uint32_t c32[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) c32[j] = 0;
    const uint32_t* src = p.in + (int64_t)bimg * p.HW * words + wi;
    // position q = t*HW + s of this image sits at ((t*B + bimg)*HW + s) * words: walked
    // incrementally (no division per word)
    int sp = slice % p.HW;
    int64_t off = ((int64_t)(slice / p.HW) * p.B * p.HW + sp) * words;
    const int64_t step = (int64_t)nslice * words, tjump = (int64_t)(p.B - 1) * p.HW * words;
    int left = (npos - slice + nslice - 1) / nslice;  // positions this thread reads
    auto advance = [&]() {
      sp += nslice;
      off += step;
      while (sp >= p.HW) {
        sp -= p.HW;
        off += tjump;
      }
    };
    while (left >= 15) {
      uint32_t by[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
      for (int r = 0; r < 17 && left >= 15; ++r) {
        uint32_t w[15];
#pragma unroll
        for (int k = 0; k < 15; ++k) {
          w[k] = src[off];
          advance();
        }
        left -= 15;
        uint32_t a = 0, b = 0, c = 0, d = 0;
#pragma unroll
        for (int k = 0; k < 15; ++k) {
          a += w[k] & 0x11111111u;
          b += (w[k] >> 1) & 0x11111111u;
          c += (w[k] >> 2) & 0x11111111u;
          d += (w[k] >> 3) & 0x11111111u;
        }
        by[0] += a & 0x0f0f0f0fu; by[1] += (a >> 4) & 0x0f0f0f0fu;
        by[2] += b & 0x0f0f0f0fu; by[3] += (b >> 4) & 0x0f0f0f0fu;
        by[4] += c & 0x0f0f0f0fu; by[5] += (c >> 4) & 0x0f0f0f0fu;
        by[6] += d & 0x0f0f0f0fu; by[7] += (d >> 4) & 0x0f0f0f0fu;
      }
      // byte m of by[2l + h] counts channel 8m + 4h + l
#pragma unroll
      for (int l = 0; l < 4; ++l)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int m = 0; m < 4; ++m) c32[8 * m + 4 * h + l] += (by[2 * l + h] >> (8 * m)) & 0xffu;
    }
    // the last < 15 positions (all of them on small grids): one add per bit
    for (; left > 0; --left) {
      const uint32_t w = src[off];
      advance();
#pragma unroll
      for (int j = 0; j < 32; ++j) c32[j] += (w >> j) & 1u;
    }
#pragma unroll
    for (int j = 0; j < 32; ++j)
      if (c32[j]) atomicAdd(&cnt[wi * 32 + j], (int)c32[j]);
  }
  __syncthreads();
  // channel c of plane pl is bit (pl*C + c) of a position's words
  for (int c = threadIdx.x; c < p.C; c += NT) {
    int sum = 0;
    for (int pl = 0; pl < planes; ++pl) sum += cnt[pl * p.C + c] << pl;
    // mean over HW then over T: both exact or one rounding for the integer sums here
    feat[c] = ((float)sum / (float)p.HW) / (float)p.T;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int nwave_out = (NT >> 6) * HEAD_OPW;  // outputs per pass of the workgroup
  for (int base = blockIdx.y * nwave_out; base < p.N_out; base += gridDim.y * nwave_out) {
    const int o0 = base + (int)(threadIdx.x >> 6) * HEAD_OPW;
    float acc[HEAD_OPW];
    const float* wrow[HEAD_OPW];
#pragma unroll
    for (int j = 0; j < HEAD_OPW; ++j) {
      acc[j] = 0.f;
      wrow[j] = p.w + (int64_t)min(o0 + j, p.N_out - 1) * p.C;  // rows past N_out: computed, not stored
    }
    // branch-free body, so the unrolled iterations' loads are all in flight together
#pragma unroll 8
    for (int c = lane; c < p.C; c += 64) {
      const float f = feat[c];
#pragma unroll
      for (int j = 0; j < HEAD_OPW; ++j) acc[j] = __builtin_fmaf(f, wrow[j][c], acc[j]);
    }
#pragma unroll
    for (int j = 0; j < HEAD_OPW; ++j) {
      const float v = wave_sum(acc[j]);
      if (lane == 0 && o0 + j < p.N_out) p.out[(int64_t)bimg * p.N_out + o0 + j] = v + p.b[o0 + j];
    }
  }
}

constexpr int kHeadMaxSplit = 64;  // summing workgroups per image (sengine_amd_sew_head_ws)

// One head launch for checked parameters (the count phase reads p.partial when set).
int launch_head(const HeadParams& p, hipStream_t stream) {
  const int T = p.T, B = p.B, HW = p.HW, C = p.C, planes = p.planes, N_out = p.N_out;
  // fp16 input (planes 0) reads 16 bits per value: weighed as 16 planes for the launch shape;
  // with precomputed sums there is nothing left to count
  const int64_t words_per_image = p.partial ? 0 : (int64_t)T * HW * (planes ? planes : 16) * C / 32;
  if (words_per_image >= 16384) {
    // counting dominates (token grids): one 1024-thread workgroup per image counts once
    hipLaunchKernelGGL(sew_head_kernel<1024>, dim3((unsigned)B, 1u), dim3(1024), 0, stream, p);
  } else {
    // a few output slices per image (each counts its image again), so that about 512
    // workgroups share the chip
    const int passes = (N_out + 4 * HEAD_OPW - 1) / (4 * HEAD_OPW);
    const int slices = std::max(1, std::min(passes, (512 + B - 1) / B));
    hipLaunchKernelGGL(sew_head_kernel<256>, dim3((unsigned)B, (unsigned)slices), dim3(256), 0, stream, p);
  }
  return (int)hipGetLastError();
}

}  // namespace sengine

using namespace sengine;

static bool env_stem_mfma() {  // read per call: tests compare both stem kernels
  const char* e = getenv("SENGINE_AMD_STEM_MFMA");
  return !(e && atoi(e) == 0);
}

// Staged input floats of one workgroup of `pix` output pixels (at most ceil(pix / OW) + 1 rows).
static int64_t stem_staged(const StemParams& p, int pix) {
  const int64_t orows = std::min<int64_t>(p.OH, (pix + p.OW - 1) / p.OW + 1);
  return (int64_t)p.C * ((orows - 1) * p.SH + p.KH) * (p.W + 2 * p.PW);
}

// Launch geometry of stem_mfma_kernel<..., NB>: workgroups, the rounds the chip needs for
// them at the occupancy the kernel reaches (resident workgroups per CU x CUs), and its LDS.
template <int K_, int NWV, bool FASTN, int NB>
static void stem_mfma_shape(const StemParams& p, int cus, int64_t& wgs, int64_t& rounds, size_t& lds) {
  lds = (size_t)(stem_staged(p, 16 * NB) + 4 * ((3 * K_ * K_ + 3) / 4)) * sizeof(float);  // + tap offsets
  wgs = (int64_t)p.N * ((p.OH * p.OW + 16 * NB - 1) / (16 * NB));
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(
                                                       &stem_mfma_kernel<3, K_, K_, NWV, FASTN, NB>),
                                                   64 * NWV, lds) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  const int64_t slots = (int64_t)per_cu * cus;
  rounds = (wgs + slots - 1) / slots;
}

// Pixels per workgroup (16 NB): the fewest pixel-block rounds over the chip, weighing a round
// by its workgroup's pixels; at equal cost the larger block (less halo staging).
template <int K_, int NWV, bool FASTN>
static int launch_stem_mfma(const StemParams& p, hipStream_t stream) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                               hipSuccess)
    cus = 256;
  int64_t w16, r16, w11, r11, w8, r8;
  size_t l16, l11, l8;
  stem_mfma_shape<K_, NWV, FASTN, 16>(p, cus, w16, r16, l16);
  stem_mfma_shape<K_, NWV, FASTN, 11>(p, cus, w11, r11, l11);
  stem_mfma_shape<K_, NWV, FASTN, 8>(p, cus, w8, r8, l8);
  int nb = 16;
  int64_t best = r16 * 16;
  if (r11 * 11 < best) { nb = 11; best = r11 * 11; }
  if (r8 * 8 < best) nb = 8;
  if (const char* e = getenv("SENGINE_AMD_STEM_NB")) {
    const int f = atoi(e);
    if (f == 16 || f == 11 || f == 8) nb = f;
  }
  const dim3 block(64 * NWV);
  if (nb == 16)
    hipLaunchKernelGGL((stem_mfma_kernel<3, K_, K_, NWV, FASTN, 16>), dim3((unsigned)w16), block, l16, stream, p);
  else if (nb == 11)
    hipLaunchKernelGGL((stem_mfma_kernel<3, K_, K_, NWV, FASTN, 11>), dim3((unsigned)w11), block, l11, stream, p);
  else
    hipLaunchKernelGGL((stem_mfma_kernel<3, K_, K_, NWV, FASTN, 8>), dim3((unsigned)w8), block, l8, stream, p);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_stem_conv_bn(const sengine_conv_lif_desc* d, const float* x, const float* weight,
                                        int32_t w_layout, const float* bn_scale, const float* bn_bias, float* out,
                                        hipStream_t stream) {
  if (!d || !x || !weight || !bn_scale || !bn_bias || !out) return set_error(-1, "stem_conv_bn: null pointer");
  if (w_layout != SENGINE_WLAYOUT_OIHW && w_layout != SENGINE_WLAYOUT_HWIO)
    return set_error(-2, "stem_conv_bn: w_layout must be OIHW or HWIO");
  if (d->B < 1 || d->C_in < 1 || d->H < 1 || d->W < 1 || d->C_out < 1 || d->KH < 1 || d->KW < 1 || d->stride_h < 1 ||
      d->stride_w < 1 || d->pad_h < 0 || d->pad_w < 0)
    return set_error(-2, "stem_conv_bn: invalid shape fields");
  if (d->dil_h != 1 || d->dil_w != 1) return set_error(-2, "stem_conv_bn: dilation must be 1");
  StemParams p;
  p.x = x; p.w = weight; p.scale = bn_scale; p.bias = bn_bias; p.out = out;
  p.N = d->B; p.C = d->C_in; p.H = d->H; p.W = d->W; p.F = d->C_out; p.KH = d->KH; p.KW = d->KW;
  p.SH = d->stride_h; p.SW = d->stride_w; p.PH = d->pad_h; p.PW = d->pad_w;
  p.OH = (d->H + 2 * d->pad_h - d->KH) / d->stride_h + 1;
  p.OW = (d->W + 2 * d->pad_w - d->KW) / d->stride_w + 1;
  if (p.OH < 1 || p.OW < 1) return set_error(-2, "stem_conv_bn: empty output");
  const int64_t total = (int64_t)p.N * p.OH * p.OW * p.F;
  // staged rows of one block of kStemPix output pixels: at most ceil(kStemPix / OW) + 1 output rows
  const int64_t max_orows = std::min<int64_t>(p.OH, (kStemPix + p.OW - 1) / p.OW + 1);
  const int64_t staged = (int64_t)p.C * ((max_orows - 1) * p.SH + p.KH) * (p.W + 2 * p.PW);
  if (w_layout == SENGINE_WLAYOUT_HWIO && p.F % 16 == 0 && staged <= kStemLdsInput &&
      reinterpret_cast<uintptr_t>(weight) % 16 == 0) {
    const int64_t blocks = (int64_t)p.N * ((p.OH * p.OW + kStemPix - 1) / kStemPix) * (p.F / 16);
    const size_t lds = (size_t)staged * sizeof(float);
    if (p.KW == 7)
      hipLaunchKernelGGL((stem_conv_bn_lds_kernel<7, kStemOut, 16>), dim3((unsigned)blocks), dim3(kStemPix), lds,
                         stream, p);
    else if (p.KW == 3)
      hipLaunchKernelGGL((stem_conv_bn_lds_kernel<3, kStemOut, 16>), dim3((unsigned)blocks), dim3(kStemPix), lds,
                         stream, p);
    else
      hipLaunchKernelGGL((stem_conv_bn_lds_kernel<0, kStemOut, 16>), dim3((unsigned)blocks), dim3(kStemPix), lds,
                         stream, p);
  } else if (w_layout == SENGINE_WLAYOUT_HWIO)
    hipLaunchKernelGGL(stem_conv_bn_kernel<1>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(stem_conv_bn_kernel<0>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_stem_conv_bn_neuron(const sengine_conv_lif_desc* d, const float* x, const float* weight,
                                               const float* bn_scale, const float* bn_bias, float* out,
                                               uint32_t* spikes, hipStream_t stream) {
  if (!d || !x || !weight || !bn_scale || !bn_bias || !spikes)
    return set_error(-1, "stem_conv_bn_neuron: null pointer");
  if (d->B < 1 || d->C_in < 1 || d->H < 1 || d->W < 1 || d->C_out < 32 || d->C_out % 32 != 0 || d->KH < 1 ||
      d->KW < 1 || d->stride_h < 1 || d->stride_w < 1 || d->pad_h < 0 || d->pad_w < 0 || d->dil_h != 1 ||
      d->dil_w != 1)
    return set_error(-2, "stem_conv_bn_neuron: invalid shape fields (C_out % 32 == 0, dilation 1)");
  if (d->T < 1) return set_error(-2, "stem_conv_bn_neuron: T >= 1");
  if (const char* why = neuron_invalid(d->neuron, d->tau)) return set_error(-2, why);
  if (reinterpret_cast<uintptr_t>(weight) % 16 != 0)
    return set_error(-2, "stem_conv_bn_neuron: weight must be 16-byte aligned");
  StemParams p{};
  p.x = x; p.w = weight; p.scale = bn_scale; p.bias = bn_bias; p.out = out;
  p.N = d->B; p.C = d->C_in; p.H = d->H; p.W = d->W; p.F = d->C_out; p.KH = d->KH; p.KW = d->KW;
  p.SH = d->stride_h; p.SW = d->stride_w; p.PH = d->pad_h; p.PW = d->pad_w;
  p.OH = (d->H + 2 * d->pad_h - d->KH) / d->stride_h + 1;
  p.OW = (d->W + 2 * d->pad_w - d->KW) / d->stride_w + 1;
  if (p.OH < 1 || p.OW < 1) return set_error(-2, "stem_conv_bn_neuron: empty output");
  const int64_t max_orows = std::min<int64_t>(p.OH, (kStemPix + p.OW - 1) / p.OW + 1);
  const int64_t staged = (int64_t)p.C * ((max_orows - 1) * p.SH + p.KH) * (p.W + 2 * p.PW);
  if (staged > kStemLdsInput)
    return set_error(-2, "stem_conv_bn_neuron: the input rows of 256 output pixels do not fit in LDS; use "
                         "stem_conv_bn + multistep_neuron_repeat");
  p.spikes = reinterpret_cast<uint16_t*>(spikes);
  p.T = d->T;
  p.np = make_neuron_params(d->neuron, d->hard_reset, d->tau, d->v_threshold, d->v_reset);
  const size_t lds = (size_t)staged * sizeof(float);
  const int64_t pblocks = (int64_t)p.N * ((p.OH * p.OW + kStemPix - 1) / kStemPix);
  // The matrix-core kernel for the 3-channel 7x7 and 3x3 stems of 32 or 64 channels (one
  // wave per 16 channels); SENGINE_AMD_STEM_MFMA=0 keeps the FMA kernel.
  if (p.C == 3 && p.KH == p.KW && (p.KW == 7 || p.KW == 3) && (p.F == 32 || p.F == 64) && env_stem_mfma()) {
    const bool fast = p.np.hard_reset && (p.np.neuron == SENGINE_NEURON_IF ||
                                          (p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2));
    if (p.KW == 7)
      return p.F == 64 ? (fast ? launch_stem_mfma<7, 4, true>(p, stream) : launch_stem_mfma<7, 4, false>(p, stream))
                       : (fast ? launch_stem_mfma<7, 2, true>(p, stream) : launch_stem_mfma<7, 2, false>(p, stream));
    return p.F == 64 ? (fast ? launch_stem_mfma<3, 4, true>(p, stream) : launch_stem_mfma<3, 4, false>(p, stream))
                     : (fast ? launch_stem_mfma<3, 2, true>(p, stream) : launch_stem_mfma<3, 2, false>(p, stream));
  }
  const int64_t blocks = pblocks * (p.F / 16);
  if (p.KW == 7)
    hipLaunchKernelGGL((stem_conv_bn_lds_kernel<7, kStemSpikes, 16>), dim3((unsigned)blocks), dim3(kStemPix), lds,
                       stream, p);
  else if (p.KW == 3)
    hipLaunchKernelGGL((stem_conv_bn_lds_kernel<3, kStemSpikes, 16>), dim3((unsigned)blocks), dim3(kStemPix), lds,
                       stream, p);
  else
    hipLaunchKernelGGL((stem_conv_bn_lds_kernel<0, kStemSpikes, 16>), dim3((unsigned)blocks), dim3(kStemPix), lds,
                       stream, p);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_stem_conv_bn_lif_pool(const sengine_conv_lif_desc* d, const float* x, const float* weight,
                                                 const float* bn_scale, const float* bn_bias, int32_t pool_k,
                                                 int32_t pool_stride, int32_t pool_pad, uint32_t* spikes,
                                                 uint32_t* pooled, hipStream_t stream) {
  if (!d || !x || !weight || !bn_scale || !bn_bias || !pooled)
    return set_error(-1, "stem_conv_bn_lif_pool: null pointer");
  if (d->B < 1 || d->C_in < 1 || d->H < 1 || d->W < 1 || d->C_out < 16 || d->C_out % 32 != 0 || d->KH < 1 ||
      d->KW < 1 || d->stride_h < 1 || d->stride_w < 1 || d->pad_h < 0 || d->pad_w < 0 || d->dil_h != 1 ||
      d->dil_w != 1)
    return set_error(-2, "stem_conv_bn_lif_pool: invalid shape fields (C_out % 32 == 0, dilation 1)");
  if (d->T < 1 || d->T > kStemMaxT) return set_error(-2, "stem_conv_bn_lif_pool: 1 <= T <= 16");
  if (const char* why = neuron_invalid(d->neuron, d->tau)) return set_error(-2, why);
  if (pool_k < 1 || pool_stride < 1 || pool_pad < 0 || 2 * pool_pad > pool_k)
    return set_error(-2, "stem_conv_bn_lif_pool: pool needs k >= 1, stride >= 1, 0 <= pad <= k/2");
  StemParams p{};
  p.x = x; p.w = weight; p.scale = bn_scale; p.bias = bn_bias; p.out = nullptr;
  p.N = d->B; p.C = d->C_in; p.H = d->H; p.W = d->W; p.F = d->C_out; p.KH = d->KH; p.KW = d->KW;
  p.SH = d->stride_h; p.SW = d->stride_w; p.PH = d->pad_h; p.PW = d->pad_w;
  p.OH = (d->H + 2 * d->pad_h - d->KH) / d->stride_h + 1;
  p.OW = (d->W + 2 * d->pad_w - d->KW) / d->stride_w + 1;
  if (p.OH < 1 || p.OW < 1) return set_error(-2, "stem_conv_bn_lif_pool: empty output");
  p.POH = (p.OH + 2 * pool_pad - pool_k) / pool_stride + 1;
  p.POW = (p.OW + 2 * pool_pad - pool_k) / pool_stride + 1;
  if (p.POH < 1 || p.POW < 1) return set_error(-2, "stem_conv_bn_lif_pool: empty pooled output");
  // one workgroup holds a whole image's stem output for its 16 channels
  const int64_t staged = (int64_t)p.C * ((p.OH - 1) * p.SH + p.KH) * (p.W + 2 * p.PW);
  if ((int64_t)p.OH * p.OW > kStemPix || staged > kStemLdsInput)
    return set_error(-2, "stem_conv_bn_lif_pool: image too large for the fused stem (OH*OW <= 256 and the "
                         "staged input must fit in LDS); use stem_conv_bn + neuron + max-pool");
  if (reinterpret_cast<uintptr_t>(weight) % 16 != 0)
    return set_error(-2, "stem_conv_bn_lif_pool: weight must be 16-byte aligned");
  p.spikes = reinterpret_cast<uint16_t*>(spikes);
  p.pooled = reinterpret_cast<uint16_t*>(pooled);
  p.T = d->T; p.PK = pool_k; p.PS = pool_stride; p.PP = pool_pad;
  p.np = make_neuron_params(d->neuron, d->hard_reset, d->tau, d->v_threshold, d->v_reset);
  const unsigned blocks = (unsigned)(p.N * (p.F / 16));
  // staged input (padded to 4 floats) + T x kStemPix 16-bit spike words
  const size_t lds = (size_t)((staged + 3) & ~3) * sizeof(float) + (size_t)p.T * kStemPix * sizeof(uint16_t);
  if (p.KW == 7)
    hipLaunchKernelGGL((stem_conv_bn_lds_kernel<7, kStemPool, 8>), dim3(blocks), dim3(2 * kStemPix), lds, stream, p);
  else
    hipLaunchKernelGGL((stem_conv_bn_lds_kernel<0, kStemPool, 8>), dim3(blocks), dim3(2 * kStemPix), lds, stream, p);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_multistep_neuron_repeat(int32_t T, int64_t n, int32_t neuron, int32_t hard_reset,
                                                   float tau, float v_threshold, float v_reset, const float* x,
                                                   uint32_t* spikes, hipStream_t stream) {
  if (T < 1 || n < 1) return set_error(-2, "multistep_neuron_repeat: T and n must be >= 1");
  if (!x || !spikes) return set_error(-1, "multistep_neuron_repeat: null pointer");
  if (const char* why = neuron_invalid(neuron, tau)) return set_error(-2, why);
  if (n % 32 != 0) return set_error(-2, "multistep_neuron_repeat: n % 32 != 0");
  RepeatNeuronParams p{x, spikes, n, T, make_neuron_params(neuron, hard_reset, tau, v_threshold, v_reset)};
  hipLaunchKernelGGL(repeat_neuron_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_maxpool_spikes(int32_t NT, int32_t H, int32_t W, int32_t C, int32_t k, int32_t stride,
                                          int32_t pad, const uint32_t* in, uint32_t* out, hipStream_t stream) {
  if (!in || !out) return set_error(-1, "maxpool_spikes: null pointer");
  if (NT < 1 || H < 1 || W < 1 || C < 32 || C % 32 != 0 || k < 1 || stride < 1 || pad < 0 || 2 * pad >= k + 1)
    return set_error(-2, "maxpool_spikes: invalid shape (C % 32 == 0, pad < k/2 + 1)");
  PoolParams p{in, out, NT, H, W, C / 32, k, stride, pad, (H + 2 * pad - k) / stride + 1, (W + 2 * pad - k) / stride + 1};
  if (p.OH < 1 || p.OW < 1) return set_error(-2, "maxpool_spikes: empty output");
  const int64_t total = (int64_t)NT * p.OH * p.OW * p.CW;
  hipLaunchKernelGGL(maxpool_bits_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_sew_head(int32_t T, int32_t B, int32_t HW, int32_t C, int32_t planes,
                                    const uint32_t* in, const float* fc_weight, const float* fc_bias, int32_t N_out,
                                    float* out, hipStream_t stream) {
  if (!in || !fc_weight || !fc_bias || !out) return set_error(-1, "sew_head: null pointer");
  if (T < 1 || B < 1 || HW < 1 || C < 32 || C % 32 != 0 || planes < 0 || planes > kMaxPlanes || N_out < 1 ||
      (int64_t)std::max(planes, 1) * C > HEAD_MAX_PC)
    return set_error(-2, "sew_head: invalid shape (C % 32 == 0, 0 <= planes <= 5, planes * C <= 8192)");
  HeadParams p{in, fc_weight, fc_bias, out, T, B, HW, C, planes, N_out};
  return launch_head(p, stream);
}

extern "C" int sengine_amd_sew_head_ws(int32_t T, int32_t B, int32_t HW, int32_t C, int32_t planes,
                                       const uint32_t* in, const float* fc_weight, const float* fc_bias,
                                       int32_t N_out, float* out, int32_t* workspace, int64_t workspace_elems,
                                       hipStream_t stream) {
  if (planes != 0) return sengine_amd_sew_head(T, B, HW, C, planes, in, fc_weight, fc_bias, N_out, out, stream);
  if (!in || !fc_weight || !fc_bias || !out || !workspace) return set_error(-1, "sew_head_ws: null pointer");
  if (T < 1 || B < 1 || HW < 1 || C < 32 || C % 32 != 0 || C > 2048 || N_out < 1)
    return set_error(-2, "sew_head_ws: invalid shape (C % 32 == 0, C <= 2048)");
  // about 2048 summing workgroups in all, at least 64 positions each
  const int64_t P = (int64_t)T * HW;
  const int nsplit = (int)std::max<int64_t>(1, std::min<int64_t>({(int64_t)kHeadMaxSplit, (2048 + B - 1) / B, P / 64}));
  if (workspace_elems < (int64_t)B * kHeadMaxSplit * C)
    return set_error(-2, "sew_head_ws: workspace smaller than B * 64 * C int32");
  hipLaunchKernelGGL(token_sums_kernel, dim3((unsigned)nsplit, (unsigned)B), dim3(256), 0, stream,
                     reinterpret_cast<const _Float16*>(in), T, B, HW, C, nsplit, workspace);
  if (hipError_t e = hipGetLastError()) return (int)e;
  HeadParams p{in, fc_weight, fc_bias, out, T, B, HW, C, 0, N_out};
  p.partial = workspace;
  p.nsplit = nsplit;
  return launch_head(p, stream);
}
