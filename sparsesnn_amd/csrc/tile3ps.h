// Fused 2:4-sparse 3x3 Conv + BN + multi-step neuron on spike bits, persistent form (gfx950).
//
// Same operator, weight blob, halo LDS layout, SMFMAC loop and epilogue as the halo-tiled
// kernel (tile_kernel.h, KS = 3; the reference's conv2d_bn_if_interleaved_kernel,
// sengine/kernels/conv2d_bn_if_t4.py:918-1022), with workgroups that stay resident: each owns
// one 64-channel block and walks a strided sequence of spatial tiles.  The (tile, chunk) steps
// of its sequence form one pipeline: the spike words of step f + 1 are loaded into registers
// when step f's reduction starts and expanded into the (single) LDS buffer once every wave is
// done reading it, and the A operands of step f + 1's first tap are loaded during step f's last
// tap, so a tile's staging latency is hidden behind the previous tile's SMFMACs and epilogue
// instead of opening every workgroup's life.
//
// Restricted to the fast launches: T = 4, one 64-channel group per wave, no reduction split,
// one-tap operand prefetch, spike bits in and out, a hard-reset LIF or IF without traces or
// residual.  STATE: the membrane state of the reference's call (V0 read, final membrane
// written; lean_epilogue_state), else V0 = 0 and the final membrane is not kept.
//
// PAIR: the input's last 64-channel chunk holds 32 real channels (a 96- or 160-channel layer
// padded to a multiple of 64; the upper 32 are zero and have no weights).  That chunk runs 5
// reduction steps instead of 9: step i takes the 32 real channels of taps 2i and 2i + 1 (tap 8
// alone, its upper half against zero weights), the lower 32 reduction slots from the first
// tap's pixel and the upper 32 from the second's.  The blob (compress_2_4_kernel, tail form)
// holds 9 * (nchunk - 1) full chunks in (tap, chunk) order, then the 5 paired chunks.
#pragma once
#include "tile_kernel.h"

namespace sengine {

template <int TR, int TC, int GR, int MODE, bool STATE, bool PAIR = false>
__global__ __launch_bounds__((TileGeom<3, TR, TC, GR>::NTHR)) __attribute__((amdgpu_waves_per_eu(3)))
void fused_tile3ps_kernel(TileParams p, int ncb) {
  using Gm = TileGeom<3, TR, TC, GR>;
  constexpr int T = 4;
  constexpr int NPIX = Gm::NPIX;
  constexpr int NTHR = Gm::NTHR;
  constexpr int UNITS = T * NPIX;                 // (t, pixel) spike words per chunk
  constexpr int UPT = (UNITS + NTHR - 1) / NTHR;  // per thread
  constexpr int PAD = Gm::PAD;
  constexpr int TS = Gm::TS;
  static_assert(MODE == EPI_LIF_HARD || MODE == EPI_IF_HARD, "fast hard-reset modes only");
  __shared__ uint2 sB[T * TS];
  __shared__ float sCoef[4][64];

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int col = lane & 15;

  // workgroup -> (channel block Gb, first tile j0); tiles j0, j0 + J, j0 + 2J, ...
  const int L = tile_remap(blockIdx.x, gridDim.x);
  const int Gb = L % ncb;
  const int j0 = L / ncb;
  const int J = (int)gridDim.x / ncb;  // host: gridDim.x % ncb == 0, J <= ntiles
  const int ntile = (p.ntiles - j0 + J - 1) / J;
  const int nf = ntile * p.nchunk;

  if (tid < 64) {
    const float sc = p.scale[Gb * 64 + tid] * p.enc_scale;  // exact: enc_scale is a power of two
    const float bi = p.bias[Gb * 64 + tid];
    const bool fold = MODE == EPI_LIF_HARD;
    sCoef[0][tid] = fold ? sc * p.np.rtau : sc;  // exact: rtau is a power of two
    sCoef[1][tid] = fold ? bi * p.np.rtau : bi;
    sCoef[2][tid] = sc;
    sCoef[3][tid] = bi;
  }

  // ---- staging identity of this thread's units u = tid + j*NTHR: (t, halo row hr, column hc)
  const int cbytes = p.C >> 3;
  int ut[UPT], uhr[UPT], uhc[UPT], soff[UPT];
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const int u = tid + j * NTHR;
    const int t = u / NPIX;
    const int px = u - t * NPIX;
    ut[j] = u < UNITS ? t : -1;
    uhr[j] = px / Gm::HC;
    uhc[j] = px - uhr[j] * Gm::HC;
    soff[j] = t * TS + px;
  }
  auto tile_origin = [&](int k, int& b, int& oh0, int& ow0) {
    const int tile = j0 + k * J;
    b = tile / p.tiles_per_image;
    const int trc = tile - b * p.tiles_per_image;
    const int tr = trc / p.tiles_w;
    oh0 = tr * TR;
    ow0 = (trc - tr * p.tiles_w) * TC;
  };
  // spike words of step f (tile f / nchunk, chunk f % nchunk); zero outside the image
  auto load_units = [&](uint2 (&v)[UPT], int f) {
    const int k = f / p.nchunk;
    const int c = f - k * p.nchunk;
    int b, oh0, ow0;
    tile_origin(k, b, oh0, ow0);
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
      const int ih = oh0 - 1 + uhr[j], iw = ow0 - 1 + uhc[j];
      const bool inb = ut[j] >= 0 && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W;
      v[j] = inb ? *reinterpret_cast<const uint2*>(p.in + (((ut[j] * p.B + b) * p.H + ih) * p.W + iw) * cbytes +
                                                  c * 8)
                 : uint2{0u, 0u};
    }
  };
  auto store_units = [&](const uint2 (&v)[UPT]) {
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
      if ((j + 1) * NTHR <= UNITS || tid + j * NTHR < UNITS) {
        u32x4_t pc[8];
        expand_word64(v[j], pc);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int q = (i >> 1) * NPIX + (i & 1) * (8 * NPIX + PAD);
          sB[soff[j] + q] = uint2{pc[i][0], pc[i][1]};
          sB[soff[j] + q + 4 * NPIX] = uint2{pc[i][2], pc[i][3]};
        }
      }
    }
  };

  // ---- compute identity: this lane's B column (halo pixel of tile-local (pr, pc))
  const int rb = wave / Gm::NCP;
  const int r_in = col >> 1;
  const int pr_ = rb * GR + r_in;
  const int pc0 = (wave - rb * Gm::NCP) * 2 + (col & 1);
  const bool pin = r_in < GR && pr_ < TR && pc0 < TC;
  const int pr = pin ? pr_ : rb * GR;  // a lane outside the tile reads a lane inside it
  const int pcl = pin ? pc0 : (pc0 < TC ? pc0 : 0);
  const int bbase = (g >> 1) * NPIX + (g & 1) * (8 * NPIX + PAD) + pr * Gm::HC + pcl;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint2*)&sB[0] + (uint32_t)bbase * 8u;

  const size_t wgroup = (size_t)p.nq * 4 * 64;
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<u32x4_t*>(p.wvals + (size_t)Gb * wgroup), 0, (int)(wgroup * sizeof(u32x4_t)), kBufferDword3);
  const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(p.wmeta + (size_t)Gb * wgroup), 0, (int)(wgroup * sizeof(uint32_t)), kBufferDword3);
  const int lv = lane * (int)sizeof(u32x4_t), lm = lane * 16;
  const int nfull = PAIR ? p.nchunk - 1 : p.nchunk;  // chunks of 64 real channels
  // A operands of chunk c's reduction step i (a tap, or in the paired chunk a tap pair)
  auto load_a = [&](int c, int i, u32x4_t (&av)[4], uint32_t (&ix)[4]) {
    const int e = ((PAIR && c == nfull) ? 9 * nfull + i : i * nfull + c) * 4 * 64;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      av[a] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                              rv, lv + a * 64 * (int)sizeof(u32x4_t), e * (int)sizeof(u32x4_t), 0));
    }
    // the lane's four tiles' metadata ([lane][tile] in the blob): one 16-byte load
    const u32x4_t m4 = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rm, lm, e * 4, 0));
#pragma unroll
    for (int a = 0; a < 4; ++a) ix[a] = m4[a];
  };

  float4_t acc[T][4];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int a = 0; a < 4; ++a) acc[t][a] = float4_t{0.f, 0.f, 0.f, 0.f};

  u32x4_t av[2][4];
  uint32_t ix[2][4];
  uint2 stg[UPT];
  if (nf > 0) {
    load_a(0, 0, av[0], ix[0]);
    load_units(stg, 0);
    store_units(stg);
  }
  __syncthreads();
  const NeuronParams np = p.np;
  const SewAdd nosew{};
  for (int f = 0; f < nf; ++f) {
    const int k = f / p.nchunk;
    const int c = f - k * p.nchunk;
    const bool more = f + 1 < nf;
    const int cn = c + 1 < p.nchunk ? c + 1 : 0;  // chunk of step f + 1
    // 9 reduction steps over this chunk (taps), or in the paired chunk 5 (tap pairs: the loop
    // leaves after step 4).  The last step uses A set 0 (9 and 5 are odd) and loads step
    // f + 1's first operands into set 1.
    const bool pc = PAIR && c == nfull;
    uint2 fr[2][4];
    // (the LDS base is an argument: asm operands do not capture through the lambda)
    auto issue = [](int step, uint2 (&fq)[4], uint32_t l0, bool pr) __attribute__((always_inline)) {
      const int i = step / T, t = step - (step / T) * T;
      const int oa = (t * TS + (i / 3) * Gm::HC + (i % 3)) * 8;
      if (PAIR && pr) {
        const int ta = 2 * i < 9 ? 2 * i : 8, tb = 2 * i + 1 < 9 ? 2 * i + 1 : 8;
        const int pa = (t * TS + (ta / 3) * Gm::HC + (ta % 3)) * 8;
        const int pb = (t * TS + (tb / 3) * Gm::HC + (tb % 3)) * 8;
        asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(fq[0]) : "v"(l0), "i"(pa));
        asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(fq[1]) : "v"(l0), "i"(pa + 4 * NPIX * 8));
        asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(fq[2]) : "v"(l0), "i"(pb));
        asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(fq[3]) : "v"(l0), "i"(pb + 4 * NPIX * 8));
      } else {
        asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(fq[0]) : "v"(l0), "i"(oa));
        asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(fq[1]) : "v"(l0), "i"(oa + 4 * NPIX * 8));
        asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(fq[2]) : "v"(l0), "i"(oa + 2 * NPIX * 8));
        asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(fq[3]) : "v"(l0), "i"(oa + 6 * NPIX * 8));
      }
    };
    issue(0, fr[0], lds0, pc);
#pragma unroll
    for (int i = 0; i < 9; ++i) {
      if (PAIR && i >= 5 && pc) continue;
      const bool last = i == 8 || (PAIR && i == 4 && pc);
      const int ra = i & 1, rn = ra ^ 1;
      if (!last) load_a(c, i + 1, av[rn], ix[rn]);
      else if (more) load_a(cn, 0, av[rn], ix[rn]);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int step = i * T + t;
        uint2(&fq)[4] = fr[step & 1];
        if (!(last && t == T - 1)) {
          issue(step + 1, fr[(step + 1) & 1], lds0, pc);
          asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(fq[0]), "+v"(fq[1]), "+v"(fq[2]), "+v"(fq[3]) :: "memory");
        } else {
          asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fq[0]), "+v"(fq[1]), "+v"(fq[2]), "+v"(fq[3]) :: "memory");
        }
        const half16_t bf = __builtin_bit_cast(
            half16_t, u32x8_t{fq[0].x, fq[0].y, fq[1].x, fq[1].y, fq[2].x, fq[2].y, fq[3].x, fq[3].y});
#pragma unroll
        for (int a = 0; a < 4; ++a)
          acc[t][a] = __builtin_amdgcn_smfmac_f32_16x16x64_f16(__builtin_bit_cast(half8_t, av[ra][a]), bf, acc[t][a],
                                                               (int)ix[ra][a], 0, 0);
      }
    }
    if (more) load_units(stg, f + 1);
    // the last step used set 0 and loaded step f + 1's first operands into set 1: move them to set 0
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      av[0][a] = av[1][a];
      ix[0][a] = ix[1][a];
    }
    if (c == p.nchunk - 1) {  // the tile's reduction is complete
      int b, oh0, ow0;
      tile_origin(k, b, oh0, ow0);
      const int oh = oh0 + pr, ow = ow0 + pcl;
      const bool valid = pin && oh < p.OH && ow < p.OW;
      const int m = valid ? (b * p.OH + oh) * p.OW + ow : 0;
      const int cl = g * 16;
      if constexpr (STATE) {
        lean_epilogue_state<MODE, SENGINE_ENC_BITS>(acc, valid, m, p.F, Gb * 64 + cl, np, &sCoef[0][cl],
                                                    &sCoef[1][cl], p.out, p.M, nosew, p.state);
      } else {
        const EpiCoeffs cf{&sCoef[0][cl], &sCoef[1][cl], &sCoef[2][cl], &sCoef[3][cl]};
        fast_epilogue_stateless<T, SENGINE_ENC_BITS, MODE>(acc, valid, m, p.M, p.F, Gb * 64 + cl, np, cf, p.out,
                                                           nosew, nullptr);
      }
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int a = 0; a < 4; ++a) acc[t][a] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
    if (more) {
      __syncthreads();  // every wave is done reading the buffer
      store_units(stg);
      __syncthreads();
    }
  }
}

// Launch on `slots` resident workgroups (all of them: with fewer, the CUs left with an extra
// workgroup would carry more tiles than any CU does now).
template <int TR, int TC, int GR, bool PAIR = false>
hipError_t launch_tile3ps(const TileParams& p, int mode, int slots, hipStream_t s) {
  const int ncb = p.F / 64;
  const int per = std::max(1, std::min(slots / ncb, p.ntiles));
  const dim3 grid((unsigned)(per * ncb)), block(TileGeom<3, TR, TC, GR>::NTHR);
  if (p.state) {
    if (mode == EPI_LIF_HARD)
      hipLaunchKernelGGL((fused_tile3ps_kernel<TR, TC, GR, EPI_LIF_HARD, true, PAIR>), grid, block, 0, s, p, ncb);
    else
      hipLaunchKernelGGL((fused_tile3ps_kernel<TR, TC, GR, EPI_IF_HARD, true, PAIR>), grid, block, 0, s, p, ncb);
  } else if (mode == EPI_LIF_HARD) {
    hipLaunchKernelGGL((fused_tile3ps_kernel<TR, TC, GR, EPI_LIF_HARD, false, PAIR>), grid, block, 0, s, p, ncb);
  } else {
    hipLaunchKernelGGL((fused_tile3ps_kernel<TR, TC, GR, EPI_IF_HARD, false, PAIR>), grid, block, 0, s, p, ncb);
  }
  return hipGetLastError();
}

}  // namespace sengine
