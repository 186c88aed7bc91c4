// Folded-BN + multi-step neuron epilogue shared by the fused kernels.
//
// One lane owns one output position m and 16 consecutive output channels cob..cob+15
// (accumulator tile a, element i -> channel cob + 4a + i, see the row permutation of the
// weight blob), for every timestep t.  The recurrence runs t = 0..T-1 in registers.
//
// MODE selects a compile-time specialisation (the epilogue's VALU work is a visible
// share of the kernel when K_red is small):
//   EPI_GENERIC  any neuron / reset / tau, optional per-step traces
//   EPI_LIF_HARD LIF with 1/tau and 1 - 1/tau powers of two (tau = 2), hard reset, no traces
//   EPI_IF_HARD  IF, hard reset, no traces
// All modes compute the same values (models/neurons.py:121-146,169-184); the fast modes
// only drop branches and fold x/tau into the BN affine (exact for power-of-two 1/tau).
#pragma once
#include "common.h"

namespace sengine {

enum { EPI_GENERIC = 0, EPI_LIF_HARD = 1, EPI_IF_HARD = 2, EPI_SHORTCUT = 3 };

// One hard-reset fire step: spike = h >= v_th (VCC), v = spike ? v_reset : h, and the spike
// shifted into `word` as its new lowest bit (word = 2*word + spike, with VCC as carry-in).
// Three VALU ops; the compiler's form needs a separate select to materialise the bit.
__device__ __forceinline__ void fire_hard(float h, float vth, float vreset, float& v, uint32_t& word) {
  asm("v_cmp_le_f32_e32 vcc, %[th], %[h]\n\t"
      "v_cndmask_b32_e32 %[v], %[h], %[vr], vcc\n\t"
      "v_addc_co_u32_e32 %[w], vcc, %[w], %[w], vcc"
      : [v] "=&v"(v), [w] "+v"(word)
      : [h] "v"(h), [th] "s"(vth), [vr] "v"(vreset)
      : "vcc");
}

// Same without the reset (last timestep, membrane not kept).
__device__ __forceinline__ void fire_only(float h, float vth, uint32_t& word) {
  asm("v_cmp_le_f32_e32 vcc, %[th], %[h]\n\t"
      "v_addc_co_u32_e32 %[w], vcc, %[w], %[w], vcc"
      : [w] "+v"(word)
      : [h] "v"(h), [th] "s"(vth)
      : "vcc");
}

// Per-lane BN coefficients for its 16 channels: folded scale/bias (x/tau folded in for the
// power-of-two LIF case, spike encoding factor folded into the scale) and the unfolded
// pair (for the BN-output trace).
struct EpiCoeffs {
  const float* fsc;
  const float* fbi;
  const float* sc;
  const float* bi;
};

// The residual words (16 channels, each plane, every t) of one lane, loaded together
// before the epilogue's t loop: the loads cannot move past the previous step's output
// stores by themselves, so loading them inside the loop costs one memory latency per t.
// Channel cob of a row is channel c of output pixel `pix` (one pixel per row unless the
// layer runs in the flat small-output layout); the planes of a pixel sit together.
constexpr int kResWords = (kMaxPlanes + 1) / 2;  // two 16-bit plane words per register

// r[t][k]: plane 2k in the low and plane 2k + 1 in the high 16 bits.
template <int T>
struct SewRes {
  uint32_t r[T][kResWords];
};

template <int T>
__device__ __forceinline__ void load_sew_res(const SewAdd& sa, int M, int m, int F, int cob, bool valid,
                                             SewRes<T>& o) {
  if (sa.res == nullptr) return;
  const int pix = cob / sa.pix_ch;
  const int c = cob - pix * sa.pix_ch;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const size_t rbase =
        ((size_t)t * M + m) * sa.res_planes * F + (size_t)pix * sa.res_planes * sa.pix_ch + c;
#pragma unroll
    for (int k = 0; k < kResWords; ++k) o.r[t][k] = 0u;
#pragma unroll
    for (int pl = 0; pl < kMaxPlanes; ++pl)
      if (valid && pl < sa.res_planes)
        o.r[t][pl >> 1] |= (uint32_t)*reinterpret_cast<const uint16_t*>(sa.res + ((rbase + (size_t)pl * sa.pix_ch) >> 3))
                           << (16 * (pl & 1));
  }
}

// Where a lane's 16 spike bits go: the output, its row width F and the lane's first channel,
// moved into the lane's plane when the output is channel-split (16 | split_c, no residual).
// Computed once before an epilogue's timestep loop; stepping plane by plane (a few planes)
// instead of dividing keeps the loop itself the same for split and unsplit outputs.
struct SpikeDst {
  uint8_t* out;
  int F;
  int cob;
};
__device__ __forceinline__ SpikeDst spike_dst(const SewAdd& sa, uint8_t* out, int F, int cob) {
  SpikeDst d{out, F, cob};
  if (sa.split_c) {
    while (d.cob >= sa.split_c) {
      d.cob -= sa.split_c;
      d.out += sa.split_bytes;
    }
    d.F = sa.split_c;
  }
  return d;
}

// Store the 16 spike bits of (position row_pos = t*M + m, channels cob..cob+15), plus the
// residual r (its planes, packed as in SewRes) when the SEW add is fused.
__device__ __forceinline__ void store_spike_word(uint32_t word, size_t row_pos, int F, int cob, uint8_t* out,
                                                 const SewAdd& sa, const uint32_t (&r)[kResWords]) {
  if (sa.res == nullptr) {
    *reinterpret_cast<uint16_t*>(out + ((row_pos * F + cob) >> 3)) = (uint16_t)word;
    return;
  }
  const int pix = cob / sa.pix_ch;
  const int c = cob - pix * sa.pix_ch;
  const size_t obase = row_pos * (size_t)sa.out_planes * F + (size_t)pix * sa.out_planes * sa.pix_ch + c;
  uint32_t carry = word;
#pragma unroll
  for (int pl = 0; pl < kMaxPlanes; ++pl) {
    if (pl >= sa.out_planes) break;
    const uint32_t rp = (r[pl >> 1] >> (16 * (pl & 1))) & 0xffffu;
    *reinterpret_cast<uint16_t*>(out + ((obase + (size_t)pl * sa.pix_ch) >> 3)) = (uint16_t)(rp ^ carry);
    carry &= rp;
  }
}

__host__ __device__ inline int epilogue_mode(const NeuronParams& np, bool traces) {
  if (traces || !np.hard_reset) return EPI_GENERIC;
  if (np.neuron == SENGINE_NEURON_LIF && np.pow2) return EPI_LIF_HARD;
  if (np.neuron == SENGINE_NEURON_IF) return EPI_IF_HARD;
  return EPI_GENERIC;
}

// The 16 spikes of a lane as fp16 0 / 1 at out + row (fp16 elements).  With a residual the
// stored value is spike + residual (exact for integers below 2048): an fp16 residual stream
// (sa.res16) at the same element, or a bit-plane residual (sa.res, its plane words r).
__device__ __forceinline__ void store_spike_f16(uint32_t word, size_t row, uint8_t* out, const SewAdd& sa,
                                                const uint32_t (&r)[kResWords]) {
  half8_t o0, o1;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    o0[j] = (word >> j) & 1u ? (_Float16)1.0f : (_Float16)0.0f;
    o1[j] = (word >> (8 + j)) & 1u ? (_Float16)1.0f : (_Float16)0.0f;
  }
  if (sa.res) {
    uint32_t val[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) val[j] = 0;
#pragma unroll
    for (int pl = 0; pl < kMaxPlanes; ++pl) {
      if (pl >= sa.res_planes) break;
      const uint32_t rp = r[pl >> 1] >> (16 * (pl & 1));
#pragma unroll
      for (int j = 0; j < 16; ++j) val[j] |= ((rp >> j) & 1u) << pl;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      o0[j] += (_Float16)(float)val[j];
      o1[j] += (_Float16)(float)val[8 + j];
    }
  }
  if (sa.res16) {
    const half8_t* r = reinterpret_cast<const half8_t*>(sa.res16 + row);
    o0 += r[0];
    o1 += r[1];
  }
  half8_t* dst = reinterpret_cast<half8_t*>(reinterpret_cast<_Float16*>(out) + row);
  dst[0] = o0;
  dst[1] = o1;
}

// Hard-reset fast modes without a state buffer: V0 = 0, so t = 0 charges h = x exactly
// (fma(0, decay, x) == x), and the membrane after the last step is not kept (no reset).
template <int T, int OUT_ENC, int MODE>
__device__ __forceinline__ void fast_epilogue_stateless(const float4_t (&acc)[T][4], bool valid, int m, int M, int F,
                                                        int cob, const NeuronParams& np, const EpiCoeffs& cf,
                                                        uint8_t* __restrict__ out, const SewAdd& sa,
                                                        const SewRes<T>* pre) {
  const SpikeDst sd = spike_dst(sa, out, F, cob);
  SewRes<T> res;
  if (pre) res = *pre;
  else load_sew_res<T>(sa, M, m, F, cob, valid, res);
  float fsc[16], fbi[16], v[16];
#pragma unroll
  for (int j = 0; j < 16; j += 4) {
    const float4_t s4 = *reinterpret_cast<const float4_t*>(cf.fsc + j);
    const float4_t b4 = *reinterpret_cast<const float4_t*>(cf.fbi + j);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      fsc[j + e] = s4[e];
      fbi[j + e] = b4[e];
    }
  }
  const float vreset = np.vreset;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 15; j >= 0; --j) {
      const float xin = __builtin_fmaf(acc[t][j >> 2][j & 3], fsc[j], fbi[j]);
      const float h = t == 0 ? xin
                             : (MODE == EPI_LIF_HARD ? __builtin_fmaf(v[j], np.decay, xin) : __fadd_rn(v[j], xin));
      if (t + 1 < T)
        fire_hard(h, np.vth, vreset, v[j], word);
      else
        fire_only(h, np.vth, word);
    }
    if (!valid) continue;
    const size_t row = ((size_t)t * M + m) * F + cob;
    if (OUT_ENC == SENGINE_ENC_BITS) {
      store_spike_word(word, (size_t)t * M + m, sd.F, sd.cob, sd.out, sa, res.r[t]);
    } else {
      store_spike_f16(word, row, out, sa, res.r[t]);
    }
  }
}

// The stateless hard-reset epilogue of fast_epilogue_stateless (T = 4) with spike bits, or fp16
// spikes plus an fp16 residual, out, reading the folded BN coefficients from LDS where they are
// used (16 registers instead of 48 held across the timesteps: the persistent kernels keep the
// next step's operands live meanwhile).  Lanes with `valid` false compute but store nothing.
// PRELOAD (fp16 output): the residual rows of all T steps are loaded before the first store --
// one memory round trip per call instead of one per step (the rows may alias the output, so a
// later step's load cannot move above an earlier step's store) -- and without a residual
// stream the same loads read the lane's own output rows and are discarded (a uniform branch
// around the loads would make the compiler's wait after the join cover the operand loads the
// persistent kernels have in flight).  32 more registers: taken by the persistent 1x1 kernel
// (Spikformer's proj and fc2 1-2 % faster), not by the direct-staged one (it would spill).
template <int MODE, int OUT_ENC, bool PRELOAD = false>
__device__ __forceinline__ void lean_epilogue_stateless(const float4_t (&acc)[4][4], bool valid, int m, int F, int cob,
                                                 const NeuronParams& np, const float* fsc, const float* fbi,
                                                 uint8_t* __restrict__ out, int M, const SewAdd& sa) {
  constexpr int T = 4;
  constexpr bool PRE = PRELOAD && OUT_ENC == SENGINE_ENC_F16;
  // Spike bits take no SEW residual here (the callers route residual layers elsewhere).
  const SpikeDst sd = spike_dst(sa, out, F, cob);
  half8_t rr[PRE ? T : 1][2];
  if constexpr (PRE) {
    const bool r16 = sa.res16 != nullptr;
    const _Float16* src = r16 ? sa.res16 : reinterpret_cast<const _Float16*>(out);
    const int mr = valid ? m : 0;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const half8_t* r = reinterpret_cast<const half8_t*>(src + ((size_t)t * M + mr) * F + cob);
      rr[t][0] = r[0];
      rr[t][1] = r[1];
    }
    if (!r16) {
#pragma unroll
      for (int t = 0; t < T; ++t) rr[t][0] = rr[t][1] = half8_t{};
    }
  }
  float v[16];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    uint32_t word = 0;
#pragma unroll
    for (int j4 = 12; j4 >= 0; j4 -= 4) {
      const float4_t s4 = *reinterpret_cast<const float4_t*>(fsc + j4);
      const float4_t b4 = *reinterpret_cast<const float4_t*>(fbi + j4);
#pragma unroll
      for (int e = 3; e >= 0; --e) {
        const int j = j4 + e;
        const float xin = __builtin_fmaf(acc[t][j >> 2][j & 3], s4[e], b4[e]);
        const float h = t == 0 ? xin
                               : (MODE == EPI_LIF_HARD ? __builtin_fmaf(v[j], np.decay, xin) : __fadd_rn(v[j], xin));
        if (t + 1 < T)
          fire_hard(h, np.vth, np.vreset, v[j], word);
        else
          fire_only(h, np.vth, word);
      }
    }
    if (!valid) continue;
    if constexpr (OUT_ENC == SENGINE_ENC_BITS) {
      *reinterpret_cast<uint16_t*>(sd.out + ((((size_t)t * M + m) * sd.F + sd.cob) >> 3)) = (uint16_t)word;
    } else if constexpr (PRE) {
      half8_t o0 = rr[t][0], o1 = rr[t][1];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        o0[j] += (word >> j) & 1u ? (_Float16)1.0f : (_Float16)0.0f;
        o1[j] += (word >> (8 + j)) & 1u ? (_Float16)1.0f : (_Float16)0.0f;
      }
      half8_t* dst = reinterpret_cast<half8_t*>(reinterpret_cast<_Float16*>(out) + ((size_t)t * M + m) * F + cob);
      dst[0] = o0;
      dst[1] = o1;
    } else {
      const uint32_t zr[kResWords] = {};
      store_spike_f16(word, ((size_t)t * M + m) * F + cob, out, sa, zr);
    }
  }
}

// lean_epilogue_stateless with a membrane state, for the persistent kernels (the reference
// executor always binds one, sengine/csrc/cpp_executor.cu:704-718,909-913): V0 is read from
// state (fp32, F channels per position: the runtime's (B*OH*OW, C_out) membrane,
// sengine/cuda_graph_runtime.py:385-390; the lane's 16 channels are 64 contiguous bytes), every
// step charges from the carried membrane and resets, and the membrane after step T - 1 is
// written back.  Same arithmetic as lif_epilogue's branch-free hard-reset loop.  Lanes with
// `valid` false compute but load and store nothing.
template <int MODE, int OUT_ENC>
__device__ __forceinline__ void lean_epilogue_state(const float4_t (&acc)[4][4], bool valid, int m, int F, int cob,
                                                    const NeuronParams& np, const float* fsc, const float* fbi,
                                                    uint8_t* __restrict__ out, int M, const SewAdd& sa, float* state) {
  constexpr int T = 4;
  const SpikeDst sd = spike_dst(sa, out, F, cob);
  float* st = state + (size_t)m * F + cob;
  float v[16];
#pragma unroll
  for (int j = 0; j < 16; j += 4) {
    const float4_t v4 = valid ? *reinterpret_cast<const float4_t*>(st + j) : float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) v[j + e] = v4[e];
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    uint32_t word = 0;
#pragma unroll
    for (int j4 = 12; j4 >= 0; j4 -= 4) {
      const float4_t s4 = *reinterpret_cast<const float4_t*>(fsc + j4);
      const float4_t b4 = *reinterpret_cast<const float4_t*>(fbi + j4);
#pragma unroll
      for (int e = 3; e >= 0; --e) {
        const int j = j4 + e;
        const float xin = __builtin_fmaf(acc[t][j >> 2][j & 3], s4[e], b4[e]);
        const float h = MODE == EPI_LIF_HARD ? __builtin_fmaf(v[j], np.decay, xin) : __fadd_rn(v[j], xin);
        fire_hard(h, np.vth, np.vreset, v[j], word);
      }
    }
    if (!valid) continue;
    if (OUT_ENC == SENGINE_ENC_BITS) {
      *reinterpret_cast<uint16_t*>(sd.out + ((((size_t)t * M + m) * sd.F + sd.cob) >> 3)) = (uint16_t)word;
    } else {
      const uint32_t zr[kResWords] = {};
      store_spike_f16(word, ((size_t)t * M + m) * F + cob, out, sa, zr);
    }
  }
  if (valid) {
#pragma unroll
    for (int j = 0; j < 16; j += 4) *reinterpret_cast<float4_t*>(st + j) = float4_t{v[j], v[j + 1], v[j + 2], v[j + 3]};
  }
}

// 4x4 transpose of 16-byte chunks across the four 16-lane rows of a wave: afterwards chunk q of
// row r holds what chunk r of row q held (rows r = lane / 16).  Two v_permlane32_swap and two
// v_permlane16_swap (gfx950) per dword position; every lane of the wave must execute it.
__device__ __forceinline__ void transpose_rows4(float4_t (&x)[4]) {
  // (through whole-vector integer copies: the swap builtins fed with per-element float bit
  // casts were compiled into wrong code by this toolchain; this form is checked on the GPU)
  uint32_t a[4][4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const u32x4_t w = __builtin_bit_cast(u32x4_t, x[q]);
#pragma unroll
    for (int e = 0; e < 4; ++e) a[q][e] = w[e];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    // rows 2, 3 of chunks 0 / 1 <-> rows 0, 1 of chunks 2 / 3
    auto s02 = __builtin_amdgcn_permlane32_swap(a[0][e], a[2][e], false, false);
    auto s13 = __builtin_amdgcn_permlane32_swap(a[1][e], a[3][e], false, false);
    // odd rows of the first <-> even rows of the second
    auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
    auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
    a[0][e] = s01[0];
    a[1][e] = s01[1];
    a[2][e] = s23[0];
    a[3][e] = s23[1];
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) x[q] = __builtin_bit_cast(float4_t, u32x4_t{a[q][0], a[q][1], a[q][2], a[q][3]});
}

// Membrane-shortcut form with bit output and no traces (EPI_SHORTCUT): y = BN(acc) + residual
// (fp32 rows, rounded once as torch's out + sc) is stored and the neuron runs on y (times 1/tau
// when folded), with an optional membrane state.  Same values as the generic path; written for
// three waves per SIMD: one timestep's residual rows are in flight while the previous step is
// computed and stored (a later step's rows are never written by an earlier step's stores, so
// the prefetch is safe when the residual and output rows alias), the BN coefficients are read
// from LDS where used.  Rows move as whole 64-byte lines when all lanes are active and every
// position's four lanes agree (see transpose_rows4).
template <int T, int OUT_ENC>
__device__ __forceinline__ void shortcut_epilogue(const float4_t (&acc)[T][4], bool valid, int m, int M, int F, int cob,
                                                  const NeuronParams& np, const EpiCoeffs& cf, float* state,
                                                  uint8_t* __restrict__ out, const SewAdd& sa) {
  const SpikeDst sd = spike_dst(sa, out, F, cob);
  const bool fold = np.neuron == SENGINE_NEURON_LIF && np.pow2;
  float v[16];
  float* st = state ? state + (size_t)m * F + cob : nullptr;
#pragma unroll
  for (int j = 0; j < 16; j += 4) {
    float4_t v4 = float4_t{0.f, 0.f, 0.f, 0.f};
    if (st && valid) v4 = *reinterpret_cast<const float4_t*>(st + j);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[j + e] = v4[e];
  }
  const int g4 = (int)(threadIdx.x & 63) >> 4;
  const int mv = valid ? m : -1;
  const bool rowwise = __builtin_amdgcn_read_exec() == ~0ull &&
                       __all((cob & 63) == 16 * g4 && __shfl_xor(mv, 16) == mv && __shfl_xor(mv, 32) == mv);
  const int cq = rowwise ? 16 : 4;
  const int c0 = rowwise ? cob - 12 * g4 : cob;
  auto load_rows = [&](int t, float4_t (&r)[4]) {
    const size_t row = ((size_t)t * M + m) * F + c0;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      r[q] = (valid && sa.real_res) ? *reinterpret_cast<const float4_t*>(sa.real_res + row + cq * q)
                                    : float4_t{0.f, 0.f, 0.f, 0.f};
    if (rowwise) transpose_rows4(r);
  };
  float4_t cur[4], nxt[4];
  load_rows(0, cur);
  const uint32_t zres[kResWords] = {};
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if (t + 1 < T) load_rows(t + 1, nxt);
    uint32_t word = 0;
#pragma unroll
    for (int j4 = 0; j4 < 16; j4 += 4) {
      const float4_t s4 = *reinterpret_cast<const float4_t*>(cf.sc + j4);
      const float4_t b4 = *reinterpret_cast<const float4_t*>(cf.bi + j4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = j4 + e;
        const float xraw = __builtin_fmaf(acc[t][j >> 2][j & 3], s4[e], b4[e]);
        const float y = sa.real_res ? __fadd_rn(xraw, cur[j >> 2][j & 3]) : xraw;
        cur[j >> 2][j & 3] = y;
        const float h = neuron_charge(np, v[j], fold ? y * np.rtau : y);
        const bool spike = h >= np.vth;
        v[j] = neuron_reset(np, h, spike);
        word |= (uint32_t)spike << j;
      }
    }
    if (rowwise) transpose_rows4(cur);
    if (valid) {
      const size_t row = ((size_t)t * M + m) * F + c0;
#pragma unroll
      for (int q = 0; q < 4; ++q) *reinterpret_cast<float4_t*>(sa.real_out + row + cq * q) = cur[q];
      store_spike_word(word, (size_t)t * M + m, sd.F, sd.cob, sd.out, sa, zres);
    }
    if (t + 1 < T) {
#pragma unroll
      for (int q = 0; q < 4; ++q) cur[q] = nxt[q];
    }
  }
  if (st && valid) {
#pragma unroll
    for (int j = 0; j < 16; j += 4)
      *reinterpret_cast<float4_t*>(st + j) = float4_t{v[j], v[j + 1], v[j + 2], v[j + 3]};
  }
}

// `valid` false (a padding position past M) computes but stores nothing: keeping the call
// unconditional avoids a divergent branch whose join reshuffles the accumulators.  `pre`:
// residual words the kernel loaded earlier (else they are loaded here).
template <int T, int OUT_ENC, int MODE>
__device__ __forceinline__ void lif_epilogue(const float4_t (&acc)[T][4], bool valid, int m, int M, int F, int cob,
                                             const NeuronParams& np, const EpiCoeffs& cf, float* state,
                                             uint8_t* __restrict__ out, float* h_trace, float* x_trace,
                                             const SewAdd& sa, const SewRes<T>* pre = nullptr) {
  const SpikeDst sd = spike_dst(sa, out, F, cob);
  if ((MODE == EPI_LIF_HARD || MODE == EPI_IF_HARD) && state == nullptr) {  // uniform branch
    fast_epilogue_stateless<T, OUT_ENC, MODE>(acc, valid, m, M, F, cob, np, cf, out, sa, pre);
    return;
  }
  if (MODE == EPI_SHORTCUT) {
    static_assert(MODE != EPI_SHORTCUT || OUT_ENC == SENGINE_ENC_BITS, "the shortcut mode writes spike bits");
    shortcut_epilogue<T, OUT_ENC>(acc, valid, m, M, F, cob, np, cf, state, out, sa);
    return;
  }
  SewRes<T> res;
  if (pre) res = *pre;
  else load_sew_res<T>(sa, M, m, F, cob, valid, res);
  float fsc[16], fbi[16], v[16];
  const bool fold = MODE == EPI_LIF_HARD || (MODE == EPI_GENERIC && np.neuron == SENGINE_NEURON_LIF && np.pow2);
  float* st = state ? state + (size_t)m * F + cob : nullptr;
  const bool has_state = st != nullptr;
#pragma unroll
  for (int j = 0; j < 16; j += 4) {
    float4_t v4 = float4_t{0.f, 0.f, 0.f, 0.f};
    if (has_state && valid) v4 = *reinterpret_cast<const float4_t*>(st + j);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[j + e] = v4[e];
  }
  const float vreset = np.vreset;
  if (MODE == EPI_GENERIC && sa.real_out != nullptr) {  // uniform branch
    // Membrane-shortcut form (no traces): y = BN(acc) + residual is stored and the neuron
    // runs on y.  All T residual rows of the lane's channels (of 4 of them for T > 4) are
    // loaded before any is used: the stores of y could alias them, so loads issued per t
    // would each wait out one memory latency.
    constexpr int RCH = T <= 4 ? 16 : 4;  // channels whose T residual rows are loaded together
    // Whole-line access: the four lanes of a position (rows g = lane / 16 of the wave, channels
    // cob = base + 16g) read and write the position's 64 channels as 64-byte lines -- load q
    // of lane g covers channels base + 16q + 4g .. +3 -- and a 4x4 chunk transpose across the
    // rows converts between that and the accumulator layout.  Used when all 64 lanes are active
    // and every position's four lanes agree; otherwise each lane moves its own 64 contiguous bytes.
    const int g4 = (int)(threadIdx.x & 63) >> 4;
    const int mv = valid ? m : -1;
    const bool rowwise = RCH == 16 && __builtin_amdgcn_read_exec() == ~0ull &&  // the transpose reads every lane
                         __all((cob & 63) == 16 * g4 && __shfl_xor(mv, 16) == mv && __shfl_xor(mv, 32) == mv);
    const int cq = rowwise ? 16 : 4;           // channel step between a lane's loads / stores
    const int c0 = rowwise ? cob - 12 * g4 : cob;  // base + 4g (row-wise) or cob
    uint32_t words[T];
#pragma unroll
    for (int t = 0; t < T; ++t) words[t] = 0;
#pragma unroll
    for (int hf = 0; hf < 16 / RCH; ++hf) {
      float4_t rr[T][RCH / 4];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const size_t row = ((size_t)t * M + m) * F + c0 + RCH * hf;
#pragma unroll
        for (int q = 0; q < RCH / 4; ++q)
          rr[t][q] = (valid && sa.real_res) ? *reinterpret_cast<const float4_t*>(sa.real_res + row + cq * q)
                                            : float4_t{0.f, 0.f, 0.f, 0.f};
      }
      if (RCH == 16 && rowwise) {
#pragma unroll
        for (int t = 0; t < T; ++t) transpose_rows4(*reinterpret_cast<float4_t(*)[4]>(&rr[t][0]));
      }
#pragma unroll
      for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int jj = 0; jj < RCH; ++jj) {
          const int j = RCH * hf + jj;
          const float accv = acc[t][j >> 2][j & 3];
          // y = BN output + residual, rounded once as torch's out + sc; the neuron takes y
          // (times 1/tau when that is folded: an exact power-of-two scaling)
          const float xraw = __builtin_fmaf(accv, cf.sc[j], cf.bi[j]);  // unfolded BN (LDS coefficients)
          const float y = sa.real_res ? __fadd_rn(xraw, rr[t][jj >> 2][jj & 3]) : xraw;
          rr[t][jj >> 2][jj & 3] = y;
          const float h = neuron_charge(np, v[j], fold ? y * np.rtau : y);
          const bool spike = h >= np.vth;
          v[j] = neuron_reset(np, h, spike);
          words[t] |= (uint32_t)spike << j;
        }
        if (RCH == 16 && rowwise) transpose_rows4(*reinterpret_cast<float4_t(*)[4]>(&rr[t][0]));
        if (valid) {
          const size_t row = ((size_t)t * M + m) * F + c0 + RCH * hf;
#pragma unroll
          for (int q = 0; q < RCH / 4; ++q) *reinterpret_cast<float4_t*>(sa.real_out + row + cq * q) = rr[t][q];
        }
      }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if (!valid) continue;
      if (OUT_ENC == SENGINE_ENC_BITS) {
        store_spike_word(words[t], (size_t)t * M + m, sd.F, sd.cob, sd.out, sa, res.r[t]);
      } else {
        store_spike_f16(words[t], ((size_t)t * M + m) * F + cob, out, sa, res.r[t]);
      }
    }
    if (has_state && valid) {
#pragma unroll
      for (int j = 0; j < 16; j += 4)
        *reinterpret_cast<float4_t*>(st + j) = float4_t{v[j], v[j + 1], v[j + 2], v[j + 3]};
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < 16; j += 4) {
    const float4_t s4 = *reinterpret_cast<const float4_t*>(cf.fsc + j);
    const float4_t b4 = *reinterpret_cast<const float4_t*>(cf.fbi + j);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      fsc[j + e] = s4[e];
      fbi[j + e] = b4[e];
    }
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    uint32_t word = 0;
    const size_t row = ((size_t)t * M + m) * F + cob;
    if (MODE == EPI_LIF_HARD || MODE == EPI_IF_HARD) {
      // Branch-free: with no state v starts at 0 and fma(0, decay, x) == x exactly; the
      // reset is computed at every step (the last one is simply not stored).  Channels
      // 15..0 so that channel j ends in bit j of the shifted-in word.
#pragma unroll
      for (int j = 15; j >= 0; --j) {
        const float xin = __builtin_fmaf(acc[t][j >> 2][j & 3], fsc[j], fbi[j]);
        const float h = MODE == EPI_LIF_HARD ? __builtin_fmaf(v[j], np.decay, xin)  // v*decay exact: one rounding
                                             : __fadd_rn(v[j], xin);
        fire_hard(h, np.vth, vreset, v[j], word);
      }
    } else {
      float rr[16];
      const bool real = sa.real_out != nullptr && valid;
      if (real) {
#pragma unroll
        for (int j = 0; j < 16; j += 4) {
          const float4_t r4 = sa.real_res ? *reinterpret_cast<const float4_t*>(sa.real_res + row + j)
                                          : float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int e = 0; e < 4; ++e) rr[j + e] = r4[e];
        }
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float accv = acc[t][j >> 2][j & 3];
        float xin = __builtin_fmaf(accv, fsc[j], fbi[j]);
        if (real) {
          // y = BN output + residual, rounded once as torch's out + sc; the neuron takes y
          // (times 1/tau when that is folded: an exact power-of-two scaling)
          const float xraw = fold ? __builtin_fmaf(accv, cf.sc[j], cf.bi[j]) : xin;
          const float y = sa.real_res ? __fadd_rn(xraw, rr[j]) : xraw;
          rr[j] = y;
          xin = fold ? y * np.rtau : y;
        }
        const float h = neuron_charge(np, v[j], xin);
        const bool spike = h >= np.vth;
        v[j] = neuron_reset(np, h, spike);
        if (h_trace && valid) h_trace[row + j] = h;
        if (x_trace && valid) x_trace[row + j] = fold ? __builtin_fmaf(accv, cf.sc[j], cf.bi[j]) : xin;
        word |= (uint32_t)spike << j;
      }
      if (real) {
#pragma unroll
        for (int j = 0; j < 16; j += 4)
          *reinterpret_cast<float4_t*>(sa.real_out + row + j) = float4_t{rr[j], rr[j + 1], rr[j + 2], rr[j + 3]};
      }
    }
    if (!valid) continue;
    if (OUT_ENC == SENGINE_ENC_BITS) {
      store_spike_word(word, (size_t)t * M + m, sd.F, sd.cob, sd.out, sa, res.r[t]);
    } else {
      store_spike_f16(word, row, out, sa, res.r[t]);
    }
  }
  if (has_state && valid) {
#pragma unroll
    for (int j = 0; j < 16; j += 4) *reinterpret_cast<float4_t*>(st + j) = float4_t{v[j], v[j + 1], v[j + 2], v[j + 3]};
  }
}

}  // namespace sengine
