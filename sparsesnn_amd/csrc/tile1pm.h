// Fused 2:4-sparse 1x1 Conv + BN + multi-step neuron, position-major workgroups (gfx950).
//
// Same operator, weight blob and epilogue as the tile kernel's 1x1 form (tile_kernel.h,
// KS = 1; the reference's conv1x1_bn_lif / conv1x1_bn_if, sengine/kernels/
// interleaved_templates.py:28-154), with the work split the other way round:
//
//  * a workgroup owns 16 output positions (one SMFMAC column block) and 4 x 64*GPW output
//    channels; wave w computes channel block w for all 16 positions and all T;
//  * the 16 positions' input spike bits are expanded to fp16 once per workgroup, for 4 x 64
//    or 2 x 64 input channels per staging phase (CG chunks), double-buffered in LDS (one
//    barrier per phase).  With 64 positions x 128 channels per workgroup (the tile kernel),
//    a 1024-channel output re-expanded every input spike 8 times and the expansion cost as
//    much VALU time as the SMFMACs; here it is 2 times (512 channels per workgroup);
//  * consecutive workgroup ids (one XCD, one L2) hold the channel blocks of the same
//    positions, so each input pixel is fetched into one L2 and each 128-byte output row is
//    written into one L2.
//
// LDS layout of a staging phase: entry ((cc*T + t)*16 + q)*16 + pos holds half-piece q
// (channels 8*(q&7) + 4*(q>>3) .. +3 of the chunk, i.e. piece q&7, half q>>3) of position
// pos: a B fragment (half-pieces g, 8+g, 4+g, 12+g) is four ds_read_b64 whose 32-lane
// halves cover 256 consecutive bytes (every bank once).
//
// NW waves per workgroup (4, or 6 for 384-channel outputs such as Spikformer's token
// Linears).  IN_ENC = SENGINE_ENC_F16 takes fp16 activations (the reference call() ABI, or an
// integer-valued fp16 stream): a (chunk, t, position) unit is eight 16-byte pieces copied as
// they are into the same layout, and each input value is staged once per NW*64*GPW output
// channels instead of once per 64 (the 64-position tile kernel).
#pragma once
#include "tile_kernel.h"

namespace sengine {

template <int T, int GPW, int CG, int OUT_ENC, int MODE, int NW = 4, int IN_ENC = SENGINE_ENC_BITS>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(GPW == 2 || MODE == EPI_GENERIC ? 2 : 3)))
void fused_tile1pm_kernel(TileParams p) {
  constexpr int NTH = 64 * NW;             // threads per workgroup
  constexpr int NCH = 64 * GPW;            // output channels per wave
  constexpr int CE = T * 16 * 16;          // LDS entries (8 bytes) per staged chunk
  constexpr int UNITS = CG * T * 16;       // (chunk, t, position) words per staging phase
  constexpr int UPT = IN_ENC == SENGINE_ENC_BITS ? (UNITS + NTH - 1) / NTH : 1;
  constexpr int PPT = IN_ENC == SENGINE_ENC_F16 ? (UNITS * 8 + NTH - 1) / NTH : 1;  // fp16: 16-byte pieces
  static_assert(CG % 2 == 0 && CG <= 4, "the A-operand ring alternates between two register sets");
  __shared__ uint2 sB[2][CG * CE];
  __shared__ float sCoef[4][NW * NCH];

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4;
  const int col = lane & 15;

  // workgroup -> (16-position group, channel super-block); consecutive ids (one XCD) share
  // the positions
  const int nsb = p.F / (NW * NCH);
  const int L = tile_remap(blockIdx.x, gridDim.x);
  const int pg = L / nsb;
  const int sb = L - pg * nsb;
  const int m0 = pg * 16;
  const int G0 = (sb * NW + wave) * GPW;  // this wave's first 64-channel group

  const bool fold = MODE == EPI_LIF_HARD || (MODE == EPI_GENERIC && p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2);
  for (int i = tid; i < NW * NCH; i += NTH) {
    const int ch = sb * NW * NCH + i;
    const float sc = p.scale[ch] * p.enc_scale;  // exact: enc_scale is a power of two
    const float bi = p.bias[ch];
    sCoef[0][i] = fold ? sc * p.np.rtau : sc;  // exact: rtau is a power of two
    sCoef[1][i] = fold ? bi * p.np.rtau : bi;
    sCoef[2][i] = sc;
    sCoef[3][i] = bi;
  }

  // ---- staging identity: unit u = tid + j*NTH -> (chunk in phase cc, t, position pos)
  const int cbytes = p.C >> 3;
  int goff[UPT];  // byte offset of the unit's 64-bit word in phase 0; -1: zero word
  int soff[UPT];
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const int u = tid + j * NTH;
    const int pos = u & 15;
    const int t = (u >> 4) % T;
    const int cc = u / (16 * T);
    const int m = m0 + pos;
    const bool inb = u < UNITS && m < p.M;
    const int ohw = p.OH * p.OW;
    const int ib = inb ? m / ohw : 0;
    const int r = m - ib * ohw;
    const int oh = inb ? r / p.OW : 0;
    const int ih = oh * p.S, iw = (r - oh * p.OW) * p.S;
    goff[j] = inb ? (((t * p.B + ib) * p.H + ih) * p.W + iw) * cbytes + cc * 8 : -1;
    soff[j] = (cc * T + t) * 256 + pos;
  }
  // fp16 input: piece pc = tid + j*NTH is piece pc & 7 of unit pc >> 3; off16 its byte offset
  // in phase 0 (-1: zero piece), poff its half-piece entry (the other half 128 entries on)
  int off16[PPT], poff[PPT];
  if (IN_ENC == SENGINE_ENC_F16) {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int pc = tid + j * NTH;
      const int u = pc >> 3, i = pc & 7;
      const int pos = u & 15;
      const int t = (u >> 4) % T;
      const int cc = u / (16 * T);
      const int m = m0 + pos;
      const bool inb = u < UNITS && m < p.M;
      const int ohw = p.OH * p.OW;
      const int ib = inb ? m / ohw : 0;
      const int r = m - ib * ohw;
      const int oh = inb ? r / p.OW : 0;
      const int ih = oh * p.S, iw = (r - oh * p.OW) * p.S;
      off16[j] = inb ? (((t * p.B + ib) * p.H + ih) * p.W + iw) * (p.C * 2) + cc * 128 + i * 16 : -1;
      poff[j] = (cc * T + t) * 256 + pos + i * 16;
    }
  }
  auto load_pieces = [&](u32x4_t (&v)[PPT], int phase) {
#pragma unroll
    for (int j = 0; j < PPT; ++j)
      v[j] = off16[j] >= 0 ? *reinterpret_cast<const u32x4_t*>(p.in + off16[j] + phase * CG * 128)
                           : u32x4_t{0u, 0u, 0u, 0u};
  };
  auto store_pieces = [&](int buf, const u32x4_t (&v)[PPT]) {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      if ((j + 1) * NTH <= UNITS * 8 || tid + j * NTH < UNITS * 8) {
        sB[buf][poff[j]] = uint2{v[j][0], v[j][1]};
        sB[buf][poff[j] + 8 * 16] = uint2{v[j][2], v[j][3]};
      }
    }
  };
  auto load_units = [&](uint2 (&v)[UPT], int phase) {
#pragma unroll
    for (int j = 0; j < UPT; ++j)
      v[j] = goff[j] >= 0 ? *reinterpret_cast<const uint2*>(p.in + goff[j] + phase * CG * 8) : uint2{0u, 0u};
  };
  auto store_units = [&](int buf, const uint2 (&v)[UPT]) {
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
      if ((j + 1) * NTH <= UNITS || tid + j * NTH < UNITS) {
        u32x4_t pc[8];
        expand_word64(v[j], pc);
#pragma unroll
        for (int i = 0; i < 8; ++i) {  // piece i: half-pieces i (channels 8i..8i+3) and 8 + i (8i+4..8i+7)
          sB[buf][soff[j] + i * 16] = uint2{pc[i][0], pc[i][1]};
          sB[buf][soff[j] + (8 + i) * 16] = uint2{pc[i][2], pc[i][3]};
        }
      }
    }
  };

  // A operands (2:4 values + metadata) of this wave's channel groups through buffer resources:
  // the chunk offset is wave-uniform (scalar offset), the lane offset a fixed VGPR.
  const size_t wgroup = (size_t)p.nq * 4 * 64;
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<u32x4_t*>(p.wvals + (size_t)G0 * wgroup), 0, (int)(GPW * wgroup * sizeof(u32x4_t)), kBufferDword3);
  const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(p.wmeta + (size_t)G0 * wgroup), 0, (int)(GPW * wgroup * sizeof(uint32_t)), kBufferDword3);
  const int lv = lane * (int)sizeof(u32x4_t), lm = lane * 16;
  auto load_a = [&](int c, u32x4_t (&av)[GPW][4], uint32_t (&ix)[GPW][4]) {
    const int q = c * 4 * 64;
#pragma unroll
    for (int gg = 0; gg < GPW; ++gg)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int e = gg * (int)wgroup + q;
        av[gg][a] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                    rv, lv + a * 64 * (int)sizeof(u32x4_t), e * (int)sizeof(u32x4_t), 0));
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

  const int nphase = p.nchunk / CG;  // host: nchunk % CG == 0
  u32x4_t av[2][GPW][4];
  uint32_t ix[2][GPW][4];
  load_a(0, av[0], ix[0]);
  uint2 stg[UPT];
  // fp16: pieces two phases ahead, in two register sets (phase ph's in pst[ph & 1]): a phase's
  // loads have a whole phase of SMFMACs before the phase that stores them
  u32x4_t pst[2][PPT];
  if (IN_ENC == SENGINE_ENC_F16) {
    load_pieces(pst[0], 0);
    store_pieces(0, pst[0]);
    if (nphase > 1) load_pieces(pst[1], 1);
  } else {
    load_units(stg, 0);
    store_units(0, stg);
  }
  __syncthreads();

  // LDS byte address of this lane's half-piece g of position col in chunk slot 0, t = 0
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint2*)&sB[0][0] +
                        (uint32_t)(g * 16 + col) * 8u;
  for (int ph = 0; ph < nphase; ++ph) {
    const int buf = ph & 1;
    const bool more = ph + 1 < nphase;
    if (IN_ENC == SENGINE_ENC_F16) {
      if (ph + 2 < nphase) {  // into the set phase ph came from (stored already)
        if (ph & 1) load_pieces(pst[1], ph + 2);
        else load_pieces(pst[0], ph + 2);
      }
    } else if (more) {
      load_units(stg, ph + 1);
    }
    const uint32_t lbase = lds0 + (uint32_t)buf * (uint32_t)(CG * CE * 8);
    constexpr int NSTEP = CG * T;
    uint2 fr[2][4];
    // half-pieces g, 8 + g, 4 + g, 12 + g: +0, +8, +4, +12 rows of 16 entries
    auto issue = [&](int step, uint2 (&f)[4]) {
      const int o = step * 256 * 8;  // (cc*T + t) block of 256 entries
      asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(f[0]) : "v"(lbase), "i"(o));
      asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(f[1]) : "v"(lbase), "i"(o + 8 * 16 * 8));
      asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(f[2]) : "v"(lbase), "i"(o + 4 * 16 * 8));
      asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(f[3]) : "v"(lbase), "i"(o + 12 * 16 * 8));
    };
    issue(0, fr[0]);
#pragma unroll
    for (int cc = 0; cc < CG; ++cc) {
      const int c = ph * CG + cc;
      const int ra = cc & 1;  // compile-time: CG is even, so chunk c always uses set c & 1
      if (c + 1 < p.nchunk) load_a(c + 1, av[ra ^ 1], ix[ra ^ 1]);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int step = cc * T + t;
        uint2(&f)[4] = fr[step & 1];
        if (step + 1 < NSTEP) {
          issue(step + 1, fr[(step + 1) & 1]);
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
    }
    if (more) {
      if (IN_ENC == SENGINE_ENC_F16) {
        if (ph & 1) store_pieces(buf ^ 1, pst[0]);  // phase ph + 1 is even
        else store_pieces(buf ^ 1, pst[1]);
      } else {
        store_units(buf ^ 1, stg);
      }
    }
    __syncthreads();
  }

  const int m = m0 + col;
  const bool valid = m < p.M;
#pragma unroll
  for (int gg = 0; gg < GPW; ++gg) {
    const int cl = wave * NCH + gg * 64 + g * 16;  // workgroup-local channel of this lane's first output
    const EpiCoeffs cf{&sCoef[0][cl], &sCoef[1][cl], &sCoef[2][cl], &sCoef[3][cl]};
    lif_epilogue<T, OUT_ENC, MODE>(acc[gg], valid, valid ? m : 0, p.M, p.F, (G0 + gg) * 64 + g * 16, p.np, cf,
                                   p.state, p.out, p.h_trace, p.x_trace, p.sew);
  }
}

template <int T, int GPW, int CG, int NW = 4, int IN_ENC = SENGINE_ENC_BITS>
hipError_t launch_tile1pm(const TileParams& p, int out_enc, int mode, hipStream_t s) {
  const dim3 grid((unsigned)(((p.M + 15) / 16) * (p.F / (NW * 64 * GPW)))), block(64 * NW);
  if (out_enc == SENGINE_ENC_BITS) {
    if (mode == EPI_LIF_HARD)
      hipLaunchKernelGGL((fused_tile1pm_kernel<T, GPW, CG, SENGINE_ENC_BITS, EPI_LIF_HARD, NW, IN_ENC>), grid, block, 0,
                         s, p);
    else if (mode == EPI_IF_HARD)
      hipLaunchKernelGGL((fused_tile1pm_kernel<T, GPW, CG, SENGINE_ENC_BITS, EPI_IF_HARD, NW, IN_ENC>), grid, block, 0,
                         s, p);
    else
      hipLaunchKernelGGL((fused_tile1pm_kernel<T, GPW, CG, SENGINE_ENC_BITS, EPI_GENERIC, NW, IN_ENC>), grid, block, 0,
                         s, p);
  } else {
    hipLaunchKernelGGL((fused_tile1pm_kernel<T, GPW, CG, SENGINE_ENC_F16, EPI_GENERIC, NW, IN_ENC>), grid, block, 0, s,
                       p);
  }
  return hipGetLastError();
}

}  // namespace sengine
