// Fused 2:4-sparse 1x1 Conv + BN + multi-step neuron on fp16 activations, persistent form
// (gfx950).
//
// Same operator, weight blob, LDS layout and epilogue as the position-major kernel
// (tile1pm.h; the reference's conv1x1_bn_lif, sengine/kernels/interleaved_templates.py:95-154,
// fed the fp16 NHWC activations of its native call() ABI, cpp_executor.cu:909-913), for the
// token Linears of a spiking transformer: thousands of 16-position groups, a short reduction
// (a few 64-channel chunks) and fp16 rows 16x the size of spike bits.  One 16-position
// workgroup per (group, channel block) spends most of its life in dependent memory round
// trips (weights, first staging, the phase barriers), and the waves of a CU cannot hide them.
// Here each workgroup stays resident and walks a strided sequence of position groups of one
// channel super-block (NW waves x 64 channels):
//
//  * the reduction phases (CG = 2 chunks each) of consecutive groups form one flat sequence;
//    the fp16 pieces of phase f + 2 are loaded when phase f starts and stored into the other
//    LDS buffer when it ends (one barrier per phase), so a group's first staging overlaps the
//    previous group's SMFMACs and epilogue instead of starting cold;
//  * the A operands keep cycling through the two-set ring across group boundaries (the
//    chunk count is even, so chunk 0 of the next group lands in set 0);
//  * a group's epilogue (BN + neuron over T, spike bits stored) runs after its last phase,
//    then the accumulators are cleared for the next group;
//  * workgroup ids are remapped so the NW-wave super-blocks of the same position groups sit
//    on one XCD (their shared fp16 rows are fetched into one L2).
//
// Spike-bit inputs (IN_ENC = SENGINE_ENC_BITS: the Linears fed by spikes, proj and fc2) stage
// 8-byte words per (chunk, t, position) instead, expanded to fp16 into the same LDS layout, and
// their outputs may be fp16 spikes plus the fp16 residual stream (the reference add kernel's
// form, the transformer's residual).
//
// Restricted to what the token Linears need: T = 4, stride 1 (position m's input row is
// t*M + m), M a multiple of 16, an even chunk count, a hard-reset LIF or IF without traces,
// spike bits out or fp16 spikes (+ an fp16 residual) out.  STATE: the membrane state of the
// reference's call (V0 read, final membrane written; lean_epilogue_state), else V0 = 0 and the
// final membrane is not kept.
#pragma once
#include "tile1pm.h"

namespace sengine {

// CG: chunks per phase, chosen so every thread stages the same number of items (fp16: 2, or
// 3 for 6-wave super-blocks of 384 channels -- the host then also requires an even phase count,
// so phase f and its position in the group have the same parity; bits: as many chunks as waves).
//
// ARES = 1 (spike-bit input whose whole reduction is one phase, nchunk == CG == 4): the wave's
// A operands for all chunks (80 registers) are loaded once and stay resident, since its channel
// block never changes; the loop then issues no A-operand loads at all.
//
// NPG = 2: a group is 32 positions, two 16-position halves whose B fragments each feed the
// wave's four A tiles: every A operand loaded feeds 8 SMFMACs instead of 4 (twice the
// accumulators), which halves the A-operand traffic per SMFMAC -- for long reductions, whose A
// operands stream from L2 for every group.
template <int NW, int CG, int MODE, int IN_ENC, int OUT_ENC, int ARES = 0, bool STATE = false, int NPG = 1>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2)))
void fused_tile1ps_kernel(TileParams p, int npg, int nsb) {
  constexpr int T = 4;
  constexpr int NTH = 64 * NW;
  constexpr int GP = 16 * NPG;     // positions per group
  constexpr int LGP = NPG == 2 ? 5 : 4;
  constexpr int CE = T * GP * 16;  // LDS entries (8 bytes) per staged chunk
  constexpr bool F16IN = IN_ENC == SENGINE_ENC_F16;
  // staged items per phase: 16-byte fp16 pieces, or 8-byte spike words of (chunk, t, position)
  constexpr int ITEMS = F16IN ? CG * T * GP * 8 : CG * T * GP;
  static_assert(NPG == 1 || (NPG == 2 && ARES == 0 && !STATE), "two position groups: streamed A operands, no state");
  constexpr int PPT = ITEMS / NTH;
  constexpr int CHB = F16IN ? 128 : 8;  // bytes of one 64-channel chunk in an input row
  using Item = std::conditional_t<F16IN, u32x4_t, uint2>;
  static_assert(MODE == EPI_LIF_HARD || MODE == EPI_IF_HARD, "fast hard-reset modes only");
  static_assert(ITEMS % NTH == 0, "every thread stages the same number of items");
  __shared__ uint2 sB[2][CG * CE];
  __shared__ float sCoef[2][NW * 64];

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4;
  const int col = lane & 15;

  // workgroup -> (channel super-block sb, first group j0); groups j0, j0 + J, j0 + 2J, ...
  const int L = tile_remap(blockIdx.x, gridDim.x);
  const int sb = L % nsb;
  const int j0 = L / nsb;
  const int J = (int)gridDim.x / nsb;  // host: gridDim.x % nsb == 0, gridDim.x / nsb <= npg
  const int nblk = (npg - j0 + J - 1) / J;
  const int G0 = sb * NW + wave;  // this wave's 64-channel group

  for (int i = tid; i < NW * 64; i += NTH) {
    const int ch = sb * NW * 64 + i;
    const float sc = p.scale[ch] * p.enc_scale;
    const float bi = p.bias[ch];
    const bool fold = MODE == EPI_LIF_HARD;
    sCoef[0][i] = fold ? sc * p.np.rtau : sc;  // exact: rtau is a power of two
    sCoef[1][i] = fold ? bi * p.np.rtau : bi;
  }

  // fp16: piece q = tid + j*NTH of a phase is piece q & 7 of unit (cc, t, pos) = q >> 3, at
  // bytes cc*128 + (q & 7)*16 of row t*M + m0 + pos; bits: unit u = tid + j*NTH, at bytes cc*8
  const int64_t rowb = F16IN ? (int64_t)p.C * 2 : (int64_t)(p.C >> 3);  // bytes per input row
  int rel[PPT], poff[PPT];
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const int q = tid + j * NTH;
    const int u = F16IN ? q >> 3 : q, i = F16IN ? q & 7 : 0;
    const int pos = u & (GP - 1);
    const int t = (u >> LGP) & (T - 1);
    const int cc = u >> (LGP + 2);
    rel[j] = (int)(((int64_t)t * p.M + pos) * rowb) + cc * CHB + i * 16;
    // 256-entry blocks per (chunk, t, 16-position half); half-piece h at +16 h
    poff[j] = ((cc * T + t) * NPG + (pos >> 4)) * 256 + (pos & 15) + i * 16;
  }
  const int nphase = p.nchunk / CG;
  const int nf = nblk * nphase;
  // byte offset of flat phase f's data relative to rel[]: group j0 + (f / nphase) * J
  auto phase_base = [&](int f) -> int64_t {
    const int blk = f / nphase;
    const int ph = f - blk * nphase;
    return (int64_t)(j0 + blk * J) * GP * rowb + ph * CG * CHB;
  };
  // through a buffer resource based at the phase's data: the lane offset is one 32-bit VGPR
  auto load_pieces = [&](Item (&v)[PPT], int f) {
    const __amdgpu_buffer_rsrc_t rin = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(p.in + phase_base(f)), 0, 0x7fffffff, kBufferDword3);
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      if constexpr (F16IN)
        v[j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rin, rel[j], 0, 0));
      else
        v[j] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rin, rel[j], 0, 0));
    }
  };
  auto store_pieces = [&](int buf, const Item (&v)[PPT]) {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      if constexpr (F16IN) {
        sB[buf][poff[j]] = uint2{v[j][0], v[j][1]};
        sB[buf][poff[j] + 8 * 16] = uint2{v[j][2], v[j][3]};
      } else {
        u32x4_t pc[8];
        expand_word64(v[j], pc);
#pragma unroll
        for (int i = 0; i < 8; ++i) {  // piece i: half-pieces i (channels 8i..8i+3) and 8 + i (8i+4..8i+7)
          sB[buf][poff[j] + i * 16] = uint2{pc[i][0], pc[i][1]};
          sB[buf][poff[j] + (8 + i) * 16] = uint2{pc[i][2], pc[i][3]};
        }
      }
    }
  };

  const size_t wgroup = (size_t)p.nq * 4 * 64;
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<u32x4_t*>(p.wvals + (size_t)G0 * wgroup), 0, (int)(wgroup * sizeof(u32x4_t)), kBufferDword3);
  const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(p.wmeta + (size_t)G0 * wgroup), 0, (int)(wgroup * sizeof(uint32_t)), kBufferDword3);
  const int lv = lane * (int)sizeof(u32x4_t), lm = lane * 16;
  auto load_a = [&](int c, u32x4_t (&av)[4], uint32_t (&ix)[4]) {
    const int e = c * 4 * 64;
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

  float4_t acc[NPG][T][4];
#pragma unroll
  for (int h = 0; h < NPG; ++h)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int a = 0; a < 4; ++a) acc[h][t][a] = float4_t{0.f, 0.f, 0.f, 0.f};

  static_assert(ARES == 0 || (CG == 4 && !F16IN), "resident A operands: one 4-chunk phase of spike bits");
  constexpr int NAS = ARES ? CG : 2;  // A-operand sets: resident chunks, or the two-set ring
  u32x4_t av[NAS][4];
  uint32_t ix[NAS][4];
  Item pst[2][PPT];  // items of phase f live in set f & 1 from their load to their store
  if (nf > 0) {
    if (ARES) {
#pragma unroll
      for (int c = 0; c < NAS; ++c) load_a(c, av[c], ix[c]);
    } else {
      load_a(0, av[0], ix[0]);
    }
    load_pieces(pst[0], 0);
    store_pieces(0, pst[0]);
    if (nf > 1) load_pieces(pst[1], 1);
  }
  __syncthreads();

  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint2*)&sB[0][0] +
                        (uint32_t)(g * 16 + col) * 8u;
  const NeuronParams np = p.np;
  // one phase; PAR = f & 1 (LDS buffer and piece set) is a compile-time constant
  auto phase = [&](int f, auto par) {
    constexpr int PAR = decltype(par)::value;
    const int blk = f / nphase;
    const int ph = f - blk * nphase;
    const uint32_t lbase = lds0 + (uint32_t)PAR * (uint32_t)(CG * CE * 8);
    constexpr int NSTEP = CG * T;
    uint2 fr[2][NPG][4];
    auto issue = [&](int step, uint2 (&fs)[NPG][4]) {
#pragma unroll
      for (int h = 0; h < NPG; ++h) {
        uint2(&fq)[4] = fs[h];
        const int o = (step * NPG + h) * 256 * 8;
        asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(fq[0]) : "v"(lbase), "i"(o));
        asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(fq[1]) : "v"(lbase), "i"(o + 8 * 16 * 8));
        asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(fq[2]) : "v"(lbase), "i"(o + 4 * 16 * 8));
        asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(fq[3]) : "v"(lbase), "i"(o + 12 * 16 * 8));
      }
    };
    issue(0, fr[0]);
#pragma unroll
    for (int cc = 0; cc < CG; ++cc) {
      const int c = ph * CG + cc;
      // chunk c uses set c & 1 (ring), or set cc (resident)
      const int ra = ARES ? cc : (CG % 2 == 0 ? cc : PAR + cc) & 1;
      // Both loads below are unconditional (the operands of an existing chunk or phase when
      // there is no next one: loaded again, then unused).  Under a branch, the compiler's wait
      // counts after the join would have to cover the path with fewer loads in flight, and it
      // falls back to waiting for every outstanding load (this chunk's prefetch included).
      if (!ARES) load_a(c + 1 < p.nchunk ? c + 1 : 0, av[ra ^ 1], ix[ra ^ 1]);  // nchunk even: set 0, the next group
      // Phase f + 2's items go out after this phase's last A-operand load: vector memory counts
      // complete in issue order, so a wait for a later-issued A operand would also wait for
      // these.  Set PAR is free: phase f's own items were stored at the end of phase f - 1.
      if (cc == CG - 1) load_pieces(pst[PAR], f + 2 < nf ? f + 2 : nf - 1);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int step = cc * T + t;
        uint2(&fs)[NPG][4] = fr[step & 1];
        if (step + 1 < NSTEP) {
          issue(step + 1, fr[(step + 1) & 1]);
          // the wait names the fragment registers as operands, so every use is ordered after it
          if (NPG == 2)
            asm volatile("s_waitcnt lgkmcnt(8)" : "+v"(fs[0][0]), "+v"(fs[0][1]), "+v"(fs[0][2]), "+v"(fs[0][3]),
                         "+v"(fs[NPG - 1][0]), "+v"(fs[NPG - 1][1]), "+v"(fs[NPG - 1][2]), "+v"(fs[NPG - 1][3])::"memory");
          else
            asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(fs[0][0]), "+v"(fs[0][1]), "+v"(fs[0][2]), "+v"(fs[0][3])::"memory");
        } else {
          if (NPG == 2)
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fs[0][0]), "+v"(fs[0][1]), "+v"(fs[0][2]), "+v"(fs[0][3]),
                         "+v"(fs[NPG - 1][0]), "+v"(fs[NPG - 1][1]), "+v"(fs[NPG - 1][2]), "+v"(fs[NPG - 1][3])::"memory");
          else
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fs[0][0]), "+v"(fs[0][1]), "+v"(fs[0][2]), "+v"(fs[0][3])::"memory");
        }
#pragma unroll
        for (int h = 0; h < NPG; ++h) {
          const uint2(&fq)[4] = fs[h];
          const half16_t bf = __builtin_bit_cast(
              half16_t, u32x8_t{fq[0].x, fq[0].y, fq[1].x, fq[1].y, fq[2].x, fq[2].y, fq[3].x, fq[3].y});
#pragma unroll
          for (int a = 0; a < 4; ++a)
            acc[h][t][a] = __builtin_amdgcn_smfmac_f32_16x16x64_f16(__builtin_bit_cast(half8_t, av[ra][a]), bf,
                                                                    acc[h][t][a], (int)ix[ra][a], 0, 0);
        }
      }
    }
    if (f + 1 < nf) store_pieces(PAR ^ 1, pst[PAR ^ 1]);
    __syncthreads();
    if (ph == nphase - 1) {  // the group's reduction is complete
      const int cl = wave * 64 + g * 16;
#pragma unroll
      for (int h = 0; h < NPG; ++h) {
        const int m = (j0 + blk * J) * GP + h * 16 + col;
        if constexpr (STATE)
          lean_epilogue_state<MODE, OUT_ENC>(acc[h], true, m, p.F, G0 * 64 + g * 16, np, &sCoef[0][cl],
                                             &sCoef[1][cl], p.out, p.M, p.sew, p.state);
        else
          lean_epilogue_stateless<MODE, OUT_ENC, true>(acc[h], true, m, p.F, G0 * 64 + g * 16, np, &sCoef[0][cl],
                                                 &sCoef[1][cl], p.out, p.M, p.sew);
      }
#pragma unroll
      for (int h = 0; h < NPG; ++h)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int a = 0; a < 4; ++a) acc[h][t][a] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
  };
  for (int f = 0; f < nf; f += 2) {
    phase(f, std::integral_constant<int, 0>{});
    if (f + 1 < nf) phase(f + 1, std::integral_constant<int, 1>{});
  }
}

// Workgroups per super-block on `slots` resident workgroups (every slot: with fewer, the CUs
// left with an extra workgroup would carry more groups than any CU does otherwise).
inline int tile1ps_per(int npg, int nsb, int slots) { return std::max(1, std::min(slots / nsb, npg)); }

// Launch on `slots` resident workgroups (a multiple of the super-block count, at most one per
// (group, super-block) pair).  WITH_STATE: the instance also has a state form, taken when
// p.state is set (the host routes state-carrying calls here only for such instances).  NPG = 2:
// 32-position groups (host: 32 | M).
template <int NW, int CG, int IN_ENC, int OUT_ENC, int ARES = 0, bool WITH_STATE = false, int NPG = 1>
hipError_t launch_tile1ps(const TileParams& p, int mode, int slots, hipStream_t s) {
  const int npg = p.M / (16 * NPG);
  const int nsb = p.F / (NW * 64);
  const int per = tile1ps_per(npg, nsb, slots);
  const dim3 grid((unsigned)(per * nsb)), block(64 * NW);
  if constexpr (WITH_STATE) {
    if (p.state) {
      if (mode == EPI_LIF_HARD)
        hipLaunchKernelGGL((fused_tile1ps_kernel<NW, CG, EPI_LIF_HARD, IN_ENC, OUT_ENC, ARES, true, NPG>), grid, block,
                           0, s, p, npg, nsb);
      else
        hipLaunchKernelGGL((fused_tile1ps_kernel<NW, CG, EPI_IF_HARD, IN_ENC, OUT_ENC, ARES, true, NPG>), grid, block,
                           0, s, p, npg, nsb);
      return hipGetLastError();
    }
  }
  if (p.state) return hipErrorInvalidValue;  // no state form of this instance
  if (mode == EPI_LIF_HARD)
    hipLaunchKernelGGL((fused_tile1ps_kernel<NW, CG, EPI_LIF_HARD, IN_ENC, OUT_ENC, ARES, false, NPG>), grid, block, 0,
                       s, p, npg, nsb);
  else
    hipLaunchKernelGGL((fused_tile1ps_kernel<NW, CG, EPI_IF_HARD, IN_ENC, OUT_ENC, ARES, false, NPG>), grid, block, 0,
                       s, p, npg, nsb);
  return hipGetLastError();
}

}  // namespace sengine
