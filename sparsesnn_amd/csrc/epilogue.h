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

enum { EPI_GENERIC = 0, EPI_LIF_HARD = 1, EPI_IF_HARD = 2 };

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

// Hard-reset fast modes without a state buffer: V0 = 0, so t = 0 charges h = x exactly
// (fma(0, decay, x) == x), and the membrane after the last step is not kept (no reset).
template <int T, int OUT_ENC, int MODE>
__device__ __forceinline__ void fast_epilogue_stateless(const float4_t (&acc)[T][4], bool valid, int m, int M, int F,
                                                        int cob, const NeuronParams& np, const EpiCoeffs& cf,
                                                        uint8_t* __restrict__ out, const SewAdd& sa,
                                                        const SewRes<T>* pre) {
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
      store_spike_word(word, (size_t)t * M + m, F, cob, out, sa, res.r[t]);
    } else {
      half8_t o0, o1;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        o0[j] = (word >> j) & 1u ? (_Float16)1.0f : (_Float16)0.0f;
        o1[j] = (word >> (8 + j)) & 1u ? (_Float16)1.0f : (_Float16)0.0f;
      }
      half8_t* dst = reinterpret_cast<half8_t*>(reinterpret_cast<_Float16*>(out) + row);
      dst[0] = o0;
      dst[1] = o1;
    }
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
  if ((MODE == EPI_LIF_HARD || MODE == EPI_IF_HARD) && state == nullptr) {  // uniform branch
    fast_epilogue_stateless<T, OUT_ENC, MODE>(acc, valid, m, M, F, cob, np, cf, out, sa, pre);
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
    uint32_t words[T];
#pragma unroll
    for (int t = 0; t < T; ++t) words[t] = 0;
#pragma unroll
    for (int hf = 0; hf < 16 / RCH; ++hf) {
      float4_t rr[T][RCH / 4];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const size_t row = ((size_t)t * M + m) * F + cob + RCH * hf;
#pragma unroll
        for (int q = 0; q < RCH / 4; ++q)
          rr[t][q] = (valid && sa.real_res) ? *reinterpret_cast<const float4_t*>(sa.real_res + row + 4 * q)
                                            : float4_t{0.f, 0.f, 0.f, 0.f};
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
        if (valid) {
          const size_t row = ((size_t)t * M + m) * F + cob + RCH * hf;
#pragma unroll
          for (int q = 0; q < RCH / 4; ++q) *reinterpret_cast<float4_t*>(sa.real_out + row + 4 * q) = rr[t][q];
        }
      }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if (!valid) continue;
      if (OUT_ENC == SENGINE_ENC_BITS) {
        store_spike_word(words[t], (size_t)t * M + m, F, cob, out, sa, res.r[t]);
      } else {
        half8_t o0, o1;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          o0[j] = (words[t] >> j) & 1u ? (_Float16)1.0f : (_Float16)0.0f;
          o1[j] = (words[t] >> (8 + j)) & 1u ? (_Float16)1.0f : (_Float16)0.0f;
        }
        half8_t* dst = reinterpret_cast<half8_t*>(reinterpret_cast<_Float16*>(out) + ((size_t)t * M + m) * F + cob);
        dst[0] = o0;
        dst[1] = o1;
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
      store_spike_word(word, (size_t)t * M + m, F, cob, out, sa, res.r[t]);
    } else {
      half8_t o0, o1;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        o0[j] = (word >> j) & 1u ? (_Float16)1.0f : (_Float16)0.0f;
        o1[j] = (word >> (8 + j)) & 1u ? (_Float16)1.0f : (_Float16)0.0f;
      }
      half8_t* dst = reinterpret_cast<half8_t*>(reinterpret_cast<_Float16*>(out) + row);
      dst[0] = o0;
      dst[1] = o1;
    }
  }
  if (has_state && valid) {
#pragma unroll
    for (int j = 0; j < 16; j += 4) *reinterpret_cast<float4_t*>(st + j) = float4_t{v[j], v[j + 1], v[j + 2], v[j + 3]};
  }
}

}  // namespace sengine
