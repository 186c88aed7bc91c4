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

__host__ __device__ inline int epilogue_mode(const NeuronParams& np, bool traces) {
  if (traces || !np.hard_reset) return EPI_GENERIC;
  if (np.neuron == SENGINE_NEURON_LIF && np.pow2) return EPI_LIF_HARD;
  if (np.neuron == SENGINE_NEURON_IF) return EPI_IF_HARD;
  return EPI_GENERIC;
}

template <int T, int OUT_ENC, int MODE>
__device__ __forceinline__ void lif_epilogue(const float4_t (&acc)[T][4], int m, int M, int F, int cob,
                                             const NeuronParams& np, const float* __restrict__ scale,
                                             const float* __restrict__ bias, float enc_scale, float* state,
                                             uint8_t* __restrict__ out, float* h_trace, float* x_trace) {
  float sc[16], bi[16], fsc[16], fbi[16], v[16];
  const bool fold = MODE == EPI_LIF_HARD || (MODE == EPI_GENERIC && np.neuron == SENGINE_NEURON_LIF && np.pow2);
#pragma unroll
  for (int j = 0; j < 16; j += 4) {
    const float4_t s4 = *reinterpret_cast<const float4_t*>(scale + cob + j);
    const float4_t b4 = *reinterpret_cast<const float4_t*>(bias + cob + j);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sc[j + e] = s4[e] * enc_scale;  // exact: enc_scale is a power of two
      bi[j + e] = b4[e];
    }
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    fsc[j] = fold ? sc[j] * np.rtau : sc[j];  // exact: rtau is a power of two when fold
    fbi[j] = fold ? bi[j] * np.rtau : bi[j];
  }
  float* st = state ? state + (size_t)m * F + cob : nullptr;
  const bool has_state = st != nullptr;
  if (has_state) {
#pragma unroll
    for (int j = 0; j < 16; j += 4) {
      const float4_t v4 = *reinterpret_cast<const float4_t*>(st + j);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[j + e] = v4[e];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = 0.f;
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    uint32_t word = 0;
    const size_t row = ((size_t)t * M + m) * F + cob;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float accv = acc[t][j >> 2][j & 3];
      const float xin = __builtin_fmaf(accv, fsc[j], fbi[j]);
      float h;
      bool spike;
      if (MODE == EPI_LIF_HARD) {
        // v*decay is exact (decay a power of two): one rounding, as v*decay + x/tau
        h = (t == 0 && !has_state) ? xin : __builtin_fmaf(v[j], np.decay, xin);
        spike = h >= np.vth;
        if (t + 1 < T || has_state) v[j] = spike ? np.vreset : h;
      } else if (MODE == EPI_IF_HARD) {
        h = (t == 0 && !has_state) ? xin : __fadd_rn(v[j], xin);
        spike = h >= np.vth;
        if (t + 1 < T || has_state) v[j] = spike ? np.vreset : h;
      } else {
        h = neuron_charge(np, v[j], xin);
        spike = h >= np.vth;
        v[j] = neuron_reset(np, h, spike);
        if (h_trace) h_trace[row + j] = h;
        if (x_trace) x_trace[row + j] = fold ? __builtin_fmaf(accv, sc[j], bi[j]) : xin;
      }
      word |= (uint32_t)spike << j;
    }
    if (OUT_ENC == SENGINE_ENC_BITS) {
      *reinterpret_cast<uint16_t*>(out + (row >> 3)) = (uint16_t)word;
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
  if (has_state) {
#pragma unroll
    for (int j = 0; j < 16; j += 4) *reinterpret_cast<float4_t*>(st + j) = float4_t{v[j], v[j + 1], v[j + 2], v[j + 3]};
  }
}

}  // namespace sengine
