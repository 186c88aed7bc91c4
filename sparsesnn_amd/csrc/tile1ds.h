// Fused 2:4-sparse 1x1 Conv + BN + multi-step neuron on fp16 activations, direct-staged form
// (gfx950): weights resident in registers, activations copied into LDS by the memory pipeline.
//
// The same operator, weight blob and epilogue as the persistent 1x1 kernel (tile1ps.h; the
// reference's conv1x1_bn_lif, sengine/kernels/interleaved_templates.py:95-154, fed the fp16
// NHWC activations of its native call() ABI, cpp_executor.cu:909-913 -- in this path the token
// Linears of a spiking transformer, models/spikformer.py:103-125, 59-71).  Two of tile1ps's
// costs are removed where the reduction is short (4 or 6 chunks of 64 input channels):
//
//  * weights: a persistent workgroup's channel block never changes, so each wave loads its 64
//    channels' A operands for the whole reduction once (NCH x 20 VGPRs) and the loop issues no
//    weight loads (tile1ps reloads them one chunk ahead for every 16-position group, a round
//    trip the SMFMACs cannot cover);
//  * activations: buffer_load_dwordx4 ... lds (gfx950's 16-byte LDS DMA) writes each lane's 16
//    bytes straight into LDS, so staging takes no VGPRs, no ds_write and no VALU.  The LDS image
//    is laid out in the SMFMAC's own B-operand order: for (chunk, t), two 1 KB blocks whose slot
//    l = 16 g + col holds channels 8g..8g+7 (block 0) and 32+8g..32+8g+7 (block 1) of position
//    col, so a lane reads its fragment with two conflict-free ds_read_b128.
//
// Work assignment and pipelining: as tile1ps, each workgroup walks a strided sequence of
// 16-position groups of one channel super-block (NW waves x 64 channels, XCD-aware ids); a
// group's reduction runs in phases of CG = 2 chunks through NBUF = 3 LDS buffers, phase f + 2
// loaded while phase f computes; at a phase's start each wave waits for its own copies of that
// phase (vmcnt counts only this wave's memory operations, and loads complete in order) and the
// workgroup barrier then covers every wave's.  The epilogue (BN + neuron over T, spikes out)
// runs after a group's last phase.
//
// Restricted to: T = 4, stride 1, 16 | M, NCH = C_in / 64 in {4, 6}, a hard-reset LIF or IF
// without traces or residual, spike bits (optionally split into planes) or fp16 spikes out,
// 32-bit activation offsets.  STATE: the reference call's membrane (V0 read, final membrane
// written; lean_epilogue_state).
#pragma once
#include "tile1ps.h"

namespace sengine {

__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds_dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_dst, 16, voff, 0, 0, 0);
}

template <int NW, int NCH, int MODE, int OUT_ENC, bool STATE>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2)))
void fused_tile1ds_kernel(TileParams p, int npg, int nsb) {
  constexpr int T = 4;
  constexpr int CG = 2;                // chunks per phase
  constexpr int NBUF = 3;              // LDS phase buffers
  constexpr int PFD = NBUF - 1;        // phases in flight
  constexpr int NTH = 64 * NW;
  constexpr int NPH = NCH / CG;        // phases per group
  constexpr int NBLK = CG * T * 2;     // 1 KB blocks per phase
  constexpr int PB = NBLK * 1024;      // bytes per phase buffer
  constexpr int BPW = NBLK / NW;       // blocks each wave copies per phase
  static_assert(NCH % CG == 0 && NBLK % NW == 0, "phase layout");
  static_assert(MODE == EPI_LIF_HARD || MODE == EPI_IF_HARD, "fast hard-reset modes only");
  __shared__ __attribute__((aligned(1024))) uint8_t sB[NBUF * PB];
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
  const int G0 = sb * NW + wave;       // this wave's 64-channel group

  for (int i = tid; i < NW * 64; i += NTH) {
    const int ch = sb * NW * 64 + i;
    const float sc = p.scale[ch] * p.enc_scale;
    const float bi = p.bias[ch];
    const bool fold = MODE == EPI_LIF_HARD;
    sCoef[0][i] = fold ? sc * p.np.rtau : sc;  // exact: rtau is a power of two
    sCoef[1][i] = fold ? bi * p.np.rtau : bi;
  }
  __syncthreads();

  // the wave's A operands for every chunk, loaded once
  const size_t wgroup = (size_t)p.nq * 4 * 64;
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<u32x4_t*>(p.wvals + (size_t)G0 * wgroup), 0, (int)(wgroup * sizeof(u32x4_t)), kBufferDword3);
  const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(p.wmeta + (size_t)G0 * wgroup), 0, (int)(wgroup * sizeof(uint32_t)), kBufferDword3);
  u32x4_t av[NCH][4];
  uint32_t ix[NCH][4];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e = c * 4 * 64;
#pragma unroll
    for (int a = 0; a < 4; ++a)
      av[c][a] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                 rv, lane * 16 + a * 64 * 16, e * (int)sizeof(u32x4_t), 0));
    // the lane's four tiles' metadata ([lane][tile] in the blob): one 16-byte load
    const u32x4_t m4 = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rm, lane * 16, e * 4, 0));
#pragma unroll
    for (int a = 0; a < 4; ++a) ix[c][a] = m4[a];
  }

  // block b = wave * BPW + j of a phase: (chunk cc, timestep t, half) = (b / 8, (b / 2) % 4, b % 2);
  // lane (g, col) copies channels 8g..8g+7 (+32 for the second half) of position col
  const int rowb = p.C * 2;  // bytes per input row
  int voff[BPW];
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
    const int b = wave * BPW + j;
    const int cc = b / (2 * T), t = (b >> 1) & (T - 1), half = b & 1;
    voff[j] = (t * p.M + col) * rowb + cc * 128 + half * 64 + g * 16;
  }
  const int nf = nblk * NPH;
  uint8_t* const sbase = &sB[0];
  // copy flat phase f (group j0 + (f / NPH) * J, chunks (f % NPH) * CG ..) into buffer f % NBUF
  auto issue = [&](int f) {
    const int blk = f / NPH, ph = f - blk * NPH;
    const uint8_t* base = p.in + ((int64_t)(j0 + blk * J) * 16 * rowb + ph * CG * 128);
    const __amdgpu_buffer_rsrc_t rin =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), 0, 0x7fffffff, kBufferDword3);
    uint8_t* dst = sbase + (f % NBUF) * PB;
#pragma unroll
    for (int j = 0; j < BPW; ++j) lds_dma16(rin, dst + (wave * BPW + j) * 1024, voff[j]);
  };

  float4_t acc[T][4];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int a = 0; a < 4; ++a) acc[t][a] = float4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int s = 0; s < PFD; ++s)
    if (s < nf) issue(s);

  const uint32_t lds_sb = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)&sB[0];
  const NeuronParams np = p.np;
  for (int blk = 0; blk < nblk; ++blk) {
#pragma unroll
    for (int ph = 0; ph < NPH; ++ph) {
      const int f = blk * NPH + ph;
      // this wave's copies of phase f are done (later phases' may still be in flight) ...
      if (f + PFD - 1 < nf)
        asm volatile("s_waitcnt vmcnt(%0)" ::"i"((PFD - 1) * BPW) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      // ... and every wave's (the barrier); every wave has also finished reading phase f - 1,
      // whose buffer the copies of phase f + PFD overwrite
      __builtin_amdgcn_s_barrier();
      if (f + PFD < nf) issue(f + PFD);
      const uint32_t lbase = lds_sb + (uint32_t)((f % NBUF) * PB) + (uint32_t)lane * 16u;
      u32x4_t fr[2][2];
      auto rd = [&](int step, u32x4_t (&q)[2]) {
        const int o = step * 2 * 1024;
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(q[0]) : "v"(lbase), "i"(o));
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(q[1]) : "v"(lbase), "i"(o + 1024));
      };
      rd(0, fr[0]);
#pragma unroll
      for (int cc = 0; cc < CG; ++cc) {
        const int c = ph * CG + cc;
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const int step = cc * T + t;
          u32x4_t(&q)[2] = fr[step & 1];
          if (step + 1 < CG * T) {
            rd(step + 1, fr[(step + 1) & 1]);
            asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(q[0]), "+v"(q[1])::"memory");
          } else {
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(q[0]), "+v"(q[1])::"memory");
          }
          const half16_t bf = __builtin_bit_cast(
              half16_t, u32x8_t{q[0][0], q[0][1], q[0][2], q[0][3], q[1][0], q[1][1], q[1][2], q[1][3]});
#pragma unroll
          for (int a = 0; a < 4; ++a)
            acc[t][a] = __builtin_amdgcn_smfmac_f32_16x16x64_f16(__builtin_bit_cast(half8_t, av[c][a]), bf, acc[t][a],
                                                                 (int)ix[c][a], 0, 0);
        }
      }
    }
    // the group's reduction is complete
    const int m = (j0 + blk * J) * 16 + col;
    const int cl = wave * 64 + g * 16;
    if constexpr (STATE)
      lean_epilogue_state<MODE, OUT_ENC>(acc, true, m, p.F, G0 * 64 + g * 16, np, &sCoef[0][cl], &sCoef[1][cl],
                                         p.out, p.M, p.sew, p.state);
    else
      lean_epilogue_stateless<MODE, OUT_ENC>(acc, true, m, p.F, G0 * 64 + g * 16, np, &sCoef[0][cl], &sCoef[1][cl],
                                             p.out, p.M, p.sew);
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int a = 0; a < 4; ++a) acc[t][a] = float4_t{0.f, 0.f, 0.f, 0.f};
  }
}

// Launch on `slots` resident workgroups (a multiple of the super-block count, at most one per
// (group, super-block) pair).  p.state selects the state form.
template <int NW, int NCH, int OUT_ENC, bool WITH_STATE>
hipError_t launch_tile1ds(const TileParams& p, int mode, int slots, hipStream_t s) {
  const int npg = p.M / 16;
  const int nsb = p.F / (NW * 64);
  const int per = tile1ps_per(npg, nsb, slots);
  const dim3 grid((unsigned)(per * nsb)), block(64 * NW);
  if (p.state && !WITH_STATE) return hipErrorInvalidValue;
  if (WITH_STATE && p.state) {
    if (mode == EPI_LIF_HARD)
      hipLaunchKernelGGL((fused_tile1ds_kernel<NW, NCH, EPI_LIF_HARD, OUT_ENC, WITH_STATE>), grid, block, 0, s, p, npg,
                         nsb);
    else
      hipLaunchKernelGGL((fused_tile1ds_kernel<NW, NCH, EPI_IF_HARD, OUT_ENC, WITH_STATE>), grid, block, 0, s, p, npg,
                         nsb);
    return hipGetLastError();
  }
  if (mode == EPI_LIF_HARD)
    hipLaunchKernelGGL((fused_tile1ds_kernel<NW, NCH, EPI_LIF_HARD, OUT_ENC, false>), grid, block, 0, s, p, npg, nsb);
  else
    hipLaunchKernelGGL((fused_tile1ds_kernel<NW, NCH, EPI_IF_HARD, OUT_ENC, false>), grid, block, 0, s, p, npg, nsb);
  return hipGetLastError();
}

}  // namespace sengine
