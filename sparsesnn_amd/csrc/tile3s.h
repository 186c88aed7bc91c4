// Fused 2:4-sparse strided 3x3 Conv + BN + multi-step neuron on spike bits, halo-tiled (gfx950).
//
// The reference's conv2d_bn_if_interleaved_kernel handles any stride through its im2col
// gather (sengine/kernels/conv2d_bn_if_t4.py:918-1022, the gather at :977-992); the first conv
// of every downsampling residual block is a 3x3 / stride 2 / pad 1 conv on spikes.  Same
// operator, weight blob, SMFMAC GEMM view and epilogue as the stride-1 tile kernel
// (tile_kernel.h); what differs is the input halo.  A TR x TC output tile of stride S reads a
// ((TR-1)S+3) x ((TC-1)S+3) input halo: for S = 2 about four input pixels per output pixel,
// which as expanded fp16 (128 bytes per pixel, timestep and 64-channel chunk) would leave one
// workgroup per CU.  So the halo stays in LDS as spike bits -- 8 bytes per pixel and timestep,
// bytes interleaved [b0 b4 b1 b5 b2 b6 b3 b7] so that lane group g's 16 B-fragment bits
// (channels 8g..8g+7 and 32+8g..32+8g+7, the SMFMAC B layout) are one 16-bit word -- and every
// (tap, t) step a lane reads its word with one ds_read_u16 and expands it into the 16 fp16 B
// values in registers (17 VALU ops feeding 4 * GPW SMFMACs).  Per chunk of 64 input channels each
// input pixel is loaded from HBM once per workgroup and read by the 9 taps of every output
// pixel that covers it.
//
//  * Halo rows are padded to HCP entries so that a wave's 16 column lanes (GR x 2 output pixels,
//    stride S apart in the halo) fall on distinct LDS bank pairs for every tap: with S = 2 and
//    HCP = 18 the entries of lanes (r, c) are 2(18 r + c) + const, distinct mod 32.
//  * Chunks are double-buffered (one barrier per chunk); the spike words of a set's next chunk
//    wait in registers from the previous chunk's end (for reductions of at most two chunks per
//    set: from before the first barrier, so no HBM load sits in the in-order vector-memory queue
//    ahead of an A-operand load in the loop).
//  * A operands (2:4 values + metadata) through raw buffer resources, one tap ahead (two sets;
//    a third set two taps ahead measured no faster on any of MS-ResNet-34's strided layers).
//  * KSP = 2: a second set of waves reduces the odd chunks; accumulators are summed in LDS in a
//    fixed order before the epilogue (grids of at most one workgroup per CU).
//  * One 64-channel group per wave (GPW = 1): with two (every expanded fragment feeding 8
//    SMFMACs) the 128 accumulators, two A-operand sets and the staging registers exceed the 256
//    registers of two waves per SIMD and spill.
//  * The fast stateless epilogues run at three waves per SIMD (164-168 registers), the generic
//    one (state, traces, residuals) at two.
#pragma once
#include "tile_kernel.h"

namespace sengine {

template <int S, int TR, int TC, int GR>
struct StridedGeom {
  static constexpr int HR = (TR - 1) * S + 3;  // halo rows
  static constexpr int HC = (TC - 1) * S + 3;  // halo columns
  static constexpr int HCP = S == 2 ? 18 : HC + ((2 - HC % 4) + 4) % 4;  // padded row (see above)
  static constexpr int NPIX = HR * HCP;        // LDS entries (8 bytes) per timestep
  static constexpr int NCP = (TC + 1) / 2;
  static constexpr int NWAVE = NCP * ((TR + GR - 1) / GR);
  static constexpr int NTHR = 64 * NWAVE;
  static_assert(S != 2 || HC <= 18, "stride-2 tiles up to 8 columns");
};

// One ds_read_u16 at a compile-time byte offset from a per-lane base.
#define SENGINE_DS_READ_U16(dst, base, off) \
  asm volatile("ds_read_u16 %0, %1 offset:%2" : "=v"(dst) : "v"(base), "i"(off))

template <int S, int TR, int TC, int GR, int GPW, int OUT_ENC, int MODE, int KSP>
__global__ __launch_bounds__((StridedGeom<S, TR, TC, GR>::NTHR * KSP))
__attribute__((amdgpu_waves_per_eu(GPW == 1 && MODE != EPI_GENERIC ? 3 : 2)))
void fused_tile3s_kernel(TileParams p) {
  using Gm = StridedGeom<S, TR, TC, GR>;
  constexpr int T = 4;
  constexpr int NPIX = Gm::NPIX;
  constexpr int NTHR = Gm::NTHR;
  constexpr int UNITS = T * Gm::HR * Gm::HC;      // (t, halo pixel) spike words per chunk
  constexpr int UPT = (UNITS + NTHR - 1) / NTHR;  // per thread
  constexpr int BUFE = T * NPIX;                  // entries per buffer
  constexpr int NCH = 64 * GPW;
  __shared__ uint2 sW[KSP][2][BUFE];
  __shared__ float sCoef[4][NCH];
  // the set reduction moves one timestep's accumulators at a time through the halo buffers
  constexpr size_t kRedBytes = KSP == 2 ? (size_t)NTHR * GPW * 4 * sizeof(float4_t) : 0;
  static_assert(KSP == 1 || sizeof(sW) >= kRedBytes, "LDS too small for the set reduction");

  const int set = KSP == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)threadIdx.x / NTHR);
  const int tid = (int)threadIdx.x - set * NTHR;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int col = lane & 15;

  const int L = tile_remap(blockIdx.x, gridDim.x);
  const int Gb = L / p.ntiles;  // channel-block-major ids: an XCD's workgroups share few blocks' weights
  const int tile = L - Gb * p.ntiles;
  const int G0 = Gb * GPW;
  const int b = tile / p.tiles_per_image;
  const int trc = tile - b * p.tiles_per_image;
  const int tr = trc / p.tiles_w;
  const int oh0 = tr * TR, ow0 = (trc - tr * p.tiles_w) * TC;

  const bool fold = MODE == EPI_LIF_HARD || (MODE == EPI_GENERIC && p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2);
  if (set == 0 && tid < NCH) {
    const float sc = p.scale[G0 * 64 + tid] * p.enc_scale;  // exact: enc_scale is a power of two
    const float bi = p.bias[G0 * 64 + tid];
    sCoef[0][tid] = fold ? sc * p.np.rtau : sc;             // exact: rtau is a power of two
    sCoef[1][tid] = fold ? bi * p.np.rtau : bi;
    sCoef[2][tid] = sc;
    sCoef[3][tid] = bi;
  }

  // ---- staging identity: unit u = tid + j*NTHR -> (t, halo row hr, halo column hc)
  const int cbytes = p.C >> 3;
  int goff[UPT];  // byte offset of the unit's spike row (the host keeps the input below 2^31 bytes), -1 = zero
  int soff[UPT];  // LDS entry
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const int u = tid + j * NTHR;
    const int t = u / (Gm::HR * Gm::HC);
    const int px = u - t * (Gm::HR * Gm::HC);
    const int hr = px / Gm::HC, hc = px - hr * Gm::HC;
    const int ih = oh0 * S - 1 + hr, iw = ow0 * S - 1 + hc;
    const bool inb = u < UNITS && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W;
    goff[j] = inb ? (((t * p.B + b) * p.H + ih) * p.W + iw) * cbytes : -1;
    soff[j] = u < UNITS ? t * NPIX + hr * Gm::HCP + hc : -1;
  }
  auto load_units = [&](uint2 (&v)[UPT], int c) {
#pragma unroll
    for (int j = 0; j < UPT; ++j)
      v[j] = goff[j] >= 0 ? *reinterpret_cast<const uint2*>(p.in + goff[j] + c * 8) : uint2{0u, 0u};
  };
  auto store_units = [&](int buf, const uint2 (&v)[UPT]) {
#pragma unroll
    for (int j = 0; j < UPT; ++j)
      if ((j + 1) * NTHR <= UNITS || soff[j] >= 0) {
        // [b0 b1 b2 b3 | b4 b5 b6 b7] -> [b0 b4 b1 b5 | b2 b6 b3 b7]
        sW[set][buf][soff[j]] = uint2{__builtin_amdgcn_perm(v[j].y, v[j].x, 0x05010400u),
                                      __builtin_amdgcn_perm(v[j].y, v[j].x, 0x07030602u)};
      }
  };

  // ---- compute identity: this lane's output pixel (a lane outside the tile reads a lane inside it)
  const int rb = wave / Gm::NCP;
  const int r_in = col >> 1;
  const int pr_ = rb * GR + r_in;
  const int pc0 = (wave - rb * Gm::NCP) * 2 + (col & 1);
  const bool pin = r_in < GR && pr_ < TR && pc0 < TC;
  const int pr = pin ? pr_ : rb * GR;
  const int pc = pin ? pc0 : (pc0 < TC ? pc0 : 0);
  const int oh = oh0 + pr, ow = ow0 + pc;
  const bool valid = pin && oh < p.OH && ow < p.OW;
  const int m = valid ? (b * p.OH + oh) * p.OW + ow : 0;
  // byte address of this lane's tap-(0,0) word (lane group g's 16 bits) in buffer 0 of its set
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint2*)&sW[set][0][0] +
                        (uint32_t)(pr * S * Gm::HCP + pc * S) * 8u + 2u * (uint32_t)g;

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
      for (int a = 0; a < 4; ++a)
        av[gg][a] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rv, lv + a * 64 * (int)sizeof(u32x4_t),
                                                           (gg * (int)wgroup + q) * (int)sizeof(u32x4_t), 0));
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

  u32x4_t av[2][GPW][4];
  uint32_t ix[2][GPW][4];
  load_a(set, 0, av[0], ix[0]);  // its latency overlaps the first staging loads
  uint2 stq[UPT];  // the set's next chunk's words
  {
    uint2 stg[UPT];
    load_units(stg, set);
    if (set + KSP < p.nchunk) load_units(stq, set + KSP);
    store_units(0, stg);
  }
  __syncthreads();
  for (int c = set; c < p.nchunk; c += KSP) {  // host: nchunk % KSP == 0 (the sets stay in step)
    const bool more = c + KSP < p.nchunk;
    const int buf = (c / KSP) & 1;
    const uint32_t lbase = lds0 + (uint32_t)buf * (uint32_t)(BUFE * 8);
    // the 36 (tap, t) words, two taps ahead of their SMFMACs (waited for with an explicit
    // lgkmcnt naming the word: the loop issues no other LDS operation)
    uint32_t w[3][T];
    auto issue_tap = [&](int tp, uint32_t (&wt)[T]) {
      const int o0 = ((tp / 3) * Gm::HCP + (tp % 3)) * 8;
      SENGINE_DS_READ_U16(wt[0], lbase, o0);
      SENGINE_DS_READ_U16(wt[1], lbase, o0 + NPIX * 8);
      SENGINE_DS_READ_U16(wt[2], lbase, o0 + 2 * NPIX * 8);
      SENGINE_DS_READ_U16(wt[3], lbase, o0 + 3 * NPIX * 8);
    };
    issue_tap(0, w[0]);
    issue_tap(1, w[1]);
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      const int ra = tap & 1;
      if (tap + 1 < 9) load_a(c, tap + 1, av[ra ^ 1], ix[ra ^ 1]);
      else if (more) load_a(c + KSP, 0, av[ra ^ 1], ix[ra ^ 1]);
      if (tap + 2 < 9) issue_tap(tap + 2, w[(tap + 2) % 3]);
      uint32_t(&wt)[T] = w[tap % 3];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        // reads still in flight after this tap's word t: (T - 1 - t) of this tap, T per later tap issued
        const int later = (tap + 2 < 9 ? 2 : (tap + 1 < 9 ? 1 : 0)) * T;
        constexpr int kMaxCnt = 15;  // lgkmcnt field
        const int cnt = (T - 1 - t) + later;
        if (cnt >= kMaxCnt) asm volatile("s_waitcnt lgkmcnt(15)" : "+v"(wt[t])::"memory");
        else if (cnt == 11) asm volatile("s_waitcnt lgkmcnt(11)" : "+v"(wt[t])::"memory");
        else if (cnt == 10) asm volatile("s_waitcnt lgkmcnt(10)" : "+v"(wt[t])::"memory");
        else if (cnt == 9) asm volatile("s_waitcnt lgkmcnt(9)" : "+v"(wt[t])::"memory");
        else if (cnt == 8) asm volatile("s_waitcnt lgkmcnt(8)" : "+v"(wt[t])::"memory");
        else if (cnt == 7) asm volatile("s_waitcnt lgkmcnt(7)" : "+v"(wt[t])::"memory");
        else if (cnt == 6) asm volatile("s_waitcnt lgkmcnt(6)" : "+v"(wt[t])::"memory");
        else if (cnt == 5) asm volatile("s_waitcnt lgkmcnt(5)" : "+v"(wt[t])::"memory");
        else if (cnt == 4) asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(wt[t])::"memory");
        else if (cnt == 3) asm volatile("s_waitcnt lgkmcnt(3)" : "+v"(wt[t])::"memory");
        else if (cnt == 2) asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(wt[t])::"memory");
        else if (cnt == 1) asm volatile("s_waitcnt lgkmcnt(1)" : "+v"(wt[t])::"memory");
        else asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(wt[t])::"memory");
        const half16_t bf = expand_bits16(wt[t]);
#pragma unroll
        for (int gg = 0; gg < GPW; ++gg)
#pragma unroll
          for (int a = 0; a < 4; ++a)
            acc[gg][t][a] = __builtin_amdgcn_smfmac_f32_16x16x64_f16(__builtin_bit_cast(half8_t, av[ra][gg][a]), bf,
                                                                     acc[gg][t][a], (int)ix[ra][gg][a], 0, 0);
      }
    }
    if (more) {
      // tap 8 used set 0 and loaded the next chunk's tap 0 into set 1: move it to set 0
#pragma unroll
      for (int gg = 0; gg < GPW; ++gg)
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          av[0][gg][a] = av[1][gg][a];
          ix[0][gg][a] = ix[1][gg][a];
        }
      store_units(buf ^ 1, stq);  // the other buffer: every wave left it at the last barrier
      if (c + 2 * KSP < p.nchunk) load_units(stq, c + 2 * KSP);
      __syncthreads();
    }
  }

  if (KSP == 2) {  // set 1's accumulators join set 0's through the (now free) LDS buffers, per t
    float4_t* red = reinterpret_cast<float4_t*>(&sW[0][0][0]);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      __syncthreads();
      if (set == 1) {
#pragma unroll
        for (int gg = 0; gg < GPW; ++gg)
#pragma unroll
          for (int a = 0; a < 4; ++a) red[(gg * 4 + a) * NTHR + tid] = acc[gg][t][a];
      }
      __syncthreads();
      if (set == 0) {
#pragma unroll
        for (int gg = 0; gg < GPW; ++gg)
#pragma unroll
          for (int a = 0; a < 4; ++a) acc[gg][t][a] += red[(gg * 4 + a) * NTHR + tid];
      }
    }
    if (set == 1) return;
  }

#pragma unroll
  for (int gg = 0; gg < GPW; ++gg) {
    const int cl = gg * 64 + g * 16;  // this lane's 16 channels within the block
    const EpiCoeffs cf{&sCoef[0][cl], &sCoef[1][cl], &sCoef[2][cl], &sCoef[3][cl]};
    lif_epilogue<T, OUT_ENC, MODE>(acc[gg], valid, m, p.M, p.F, G0 * 64 + cl, p.np, cf, p.state, p.out, p.h_trace,
                                   p.x_trace, p.sew);
  }
}
#undef SENGINE_DS_READ_U16

// Tile shapes of the strided kernel: 0 = 8x8 (8-row blocks), 1 = 7x7 (7-row blocks).
template <int S, int TR, int TC, int GR, int GPW, int KSP>
hipError_t launch_tile3s_shape(const TileParams& p, int out_enc, int mode, hipStream_t s) {
  const dim3 grid((unsigned)(p.ntiles * (p.F / (64 * GPW)))), block(StridedGeom<S, TR, TC, GR>::NTHR * KSP);
  constexpr int BITS = SENGINE_ENC_BITS;
  if (out_enc == BITS) {
    if (mode == EPI_LIF_HARD)
      hipLaunchKernelGGL((fused_tile3s_kernel<S, TR, TC, GR, GPW, BITS, EPI_LIF_HARD, KSP>), grid, block, 0, s, p);
    else if (mode == EPI_IF_HARD)
      hipLaunchKernelGGL((fused_tile3s_kernel<S, TR, TC, GR, GPW, BITS, EPI_IF_HARD, KSP>), grid, block, 0, s, p);
    else
      hipLaunchKernelGGL((fused_tile3s_kernel<S, TR, TC, GR, GPW, BITS, EPI_GENERIC, KSP>), grid, block, 0, s, p);
  } else {
    hipLaunchKernelGGL((fused_tile3s_kernel<S, TR, TC, GR, GPW, SENGINE_ENC_F16, EPI_GENERIC, KSP>), grid, block,
                       0, s, p);
  }
  return hipGetLastError();
}

}  // namespace sengine
