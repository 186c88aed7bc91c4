// Spiking self-attention (Spikformer SSA, models/spikformer.py:103-130; the reference's
// TileLang matmul kernels, sengine/kernels/spikformer_kernels.py): per (t, b, head)
//     x = (Q K^T * scale) V,   then the attention neuron over T,
// with Q, K, V binary spikes (N tokens x d channels of the head).  Every product and
// partial sum is an integer (times scale, a power of two), exact in fp32 in any order, so
// this build evaluates x = Q (K^T V) * scale: K^T V is d x d, the work drops from
// N^2 d to N d^2 per head, and the result is bit-identical.
//
//   ssa_kv_kernel:     KV[t, b, h] = K^T V (int32 d x d).  A workgroup per (t*B + b, h):
//                      each wave turns 64 tokens' head slices into per-channel 64-token
//                      masks with ballots (bit transposition into LDS), then each
//                      thread sums popcount(K_i & V_j) over the token masks.
//   ssa_attend_kernel: X = Q KV on MFMA (v_mfma_f32_16x16x32_f16: A = KV^T as two exact
//                      6-bit fp16 pieces, B = Q expanded from bits), the neuron over T in
//                      registers, 16 output channels of a token assembled across lanes
//                      and stored as one u16.
#include "common.h"
#include "internal.h"

namespace sengine {

constexpr int kSsaMaxN = 8192;   // tokens (the KV kernel keeps 2 x d x N/64 token masks in LDS)
constexpr int kSsaMaxD = 64;

struct SsaParams {
  const uint32_t* q;
  const uint32_t* k;
  const uint32_t* v;
  int32_t* kv;     // (T*B, H, d, d)
  uint16_t* out;   // spike bits (T*B, N, C) viewed as u16 words
  int T, B, N, C, H, d;
  float xscale;    // scale / 2 (the MFMA sees spikes as 2.0)
  NeuronParams np;
};

// The d-bit slice of a token row (`words` u32) starting at bit `off` (off % 32 + d <= 64,
// host-checked).
__device__ __forceinline__ uint64_t head_slice(const uint32_t* row, int words, int off, int d) {
  const int w0 = off >> 5, sh = off & 31;
  const uint64_t x = ((uint64_t)(w0 + 1 < words ? row[w0 + 1] : 0u) << 32) | row[w0];
  const uint64_t v = x >> sh;
  return d == 64 ? v : (v & ((1ull << d) - 1));
}

__global__ __launch_bounds__(256) void ssa_kv_kernel(SsaParams p) {
  extern __shared__ uint64_t masks[];  // K masks [d][G], then V masks [d][G]
  const int G = (p.N + 63) >> 6;
  uint64_t* Km = masks;
  uint64_t* Vm = masks + (size_t)p.d * G;
  const int tb = blockIdx.x / p.H;
  const int h = blockIdx.x - tb * p.H;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int words = p.C >> 5;
  for (int g = wave; g < G; g += 4) {
    const int n = (g << 6) + lane;
    uint64_t ks = 0, vs = 0;
    if (n < p.N) {
      const size_t row = ((size_t)tb * p.N + n) * words;
      ks = head_slice(p.k + row, words, h * p.d, p.d);
      vs = head_slice(p.v + row, words, h * p.d, p.d);
    }
    for (int i = 0; i < p.d; ++i) {
      const uint64_t mk = __ballot((ks >> i) & 1ull);
      const uint64_t mv = __ballot((vs >> i) & 1ull);
      if (lane == 0) {
        Km[(size_t)i * G + g] = mk;
        Vm[(size_t)i * G + g] = mv;
      }
    }
  }
  __syncthreads();
  // work item = (i, 16 consecutive j): K_i masks read once per token group
  const int jchunks = p.d >> 4;
  int32_t* kv = p.kv + (size_t)blockIdx.x * p.d * p.d;
  for (int item = threadIdx.x; item < p.d * jchunks; item += blockDim.x) {
    const int i = item / jchunks;
    const int j0 = (item - i * jchunks) << 4;
    uint32_t acc[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) acc[u] = 0;
    for (int g = 0; g < G; ++g) {
      const uint64_t ki = Km[(size_t)i * G + g];
#pragma unroll
      for (int u = 0; u < 16; ++u) acc[u] += (uint32_t)__popcll(ki & Vm[(size_t)(j0 + u) * G + g]);
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) kv[i * p.d + j0 + u] = (int32_t)acc[u];
  }
}

// Workgroup = (b, h) x 64 tokens (4 waves x 16); T outer loop with the membrane in
// registers.  MFMA roles: D[j][token] = sum_i KV^T[j][i] * Q^T[i][token].
__global__ __launch_bounds__(256) void ssa_attend_kernel(SsaParams p) {
  // [piece][j][i/8]: i padded to 64 fp16 plus 8 so the 16 rows a lane group reads sit in
  // different banks
  __shared__ half8_t skv[2][kSsaMaxD][9];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int bh = blockIdx.x;
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int n = blockIdx.y * 64 + wave * 16 + c;  // this lane's token (MFMA column)
  const bool nvalid = n < p.N;
  const int words = p.C >> 5;
  const int jt_n = p.d >> 4;       // j tiles of 16
  const int ks_n = (p.d + 31) >> 5;  // k steps of 32 channels
  float v[4][4];                   // membrane per (j tile, row e)
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int e = 0; e < 4; ++e) v[jt][e] = 0.f;
  const bool fold = p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2;

  for (int t = 0; t < p.T; ++t) {
    const int tb = t * p.B + b;
    // stage KV[tb, h] as fp16 hi/lo 6-bit pieces (exact), transposed to [j][i]
    __syncthreads();
    const int32_t* kv = p.kv + ((size_t)tb * p.H + h) * p.d * p.d;
    _Float16* s = reinterpret_cast<_Float16*>(&skv[0][0][0]);
    for (int idx = threadIdx.x; idx < p.d * 64; idx += blockDim.x) {
      const int j = idx >> 6, i = idx & 63;
      const int32_t x = i < p.d ? kv[i * p.d + j] : 0;
      s[(0 * kSsaMaxD + j) * 72 + i] = (_Float16)(x & 63);
      s[(1 * kSsaMaxD + j) * 72 + i] = (_Float16)(x >> 6);
    }
    __syncthreads();
    const uint64_t qs = nvalid ? head_slice(p.q + ((size_t)tb * p.N + n) * words, words, h * p.d, p.d) : 0ull;
    float4_t lo[4], hi[4];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) lo[jt] = hi[jt] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if (ks >= ks_n) break;
      const half8_t bq = expand_bits8((uint32_t)(qs >> (32 * ks + 8 * g)) & 0xffu);
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        if (jt >= jt_n) break;
        const half8_t a0 = skv[0][jt * 16 + c][ks * 4 + g];
        const half8_t a1 = skv[1][jt * 16 + c][ks * 4 + g];
        lo[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bq, lo[jt], 0, 0, 0);
        hi[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bq, hi[jt], 0, 0, 0);
      }
    }
    // neuron on x[token][j = 16 jt + 4 g + e]; 16 spikes of a token gathered from 4 lanes
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      if (jt >= jt_n) break;
      uint32_t nib = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = __builtin_fmaf(hi[jt][e], 64.f, lo[jt][e]) * p.xscale;  // exact integers x 2^-k
        const float xf = fold ? x * p.np.rtau : x;
        const float hh = neuron_charge(p.np, v[jt][e], xf);
        const bool spike = hh >= p.np.vth;
        v[jt][e] = neuron_reset(p.np, hh, spike);
        nib |= (uint32_t)spike << e;
      }
      const uint32_t n1 = __shfl(nib, c + 16, 64), n2 = __shfl(nib, c + 32, 64), n3 = __shfl(nib, c + 48, 64);
      if (g == 0 && nvalid) {
        const uint32_t word = nib | (n1 << 4) | (n2 << 8) | (n3 << 12);
        p.out[(((size_t)tb * p.N + n) * p.C + h * p.d + jt * 16) >> 4] = (uint16_t)word;
      }
    }
  }
}

static const char* ssa_check(int T, int B, int N, int C, int H) {
  if (T < 1 || B < 1 || N < 1 || C < 32 || H < 1) return "ssa: T, B, N, heads >= 1 and C >= 32 required";
  if (N > kSsaMaxN) return "ssa: at most 8192 tokens";
  if (C % 32 != 0 || C % H != 0) return "ssa: C % 32 == 0 and C % heads == 0 required";
  const int d = C / H;
  if (d % 16 != 0 || d > kSsaMaxD) return "ssa: head dim C/heads must be a multiple of 16, at most 64";
  for (int h = 0; h < H; ++h)
    if ((h * d) % 32 + d > 64) return "ssa: head slices must sit within 64-bit windows";
  return nullptr;
}

}  // namespace sengine

using namespace sengine;

extern "C" int sengine_amd_ssa_kv(int32_t T, int32_t B, int32_t N, int32_t C, int32_t heads, const uint32_t* k_bits,
                                  const uint32_t* v_bits, int32_t* kv, hipStream_t stream) {
  if (const char* why = ssa_check(T, B, N, C, heads)) return set_error(-2, why);
  if (!k_bits || !v_bits || !kv) return set_error(-1, "ssa_kv: null pointer");
  SsaParams p{};
  p.k = k_bits; p.v = v_bits; p.kv = kv;
  p.T = T; p.B = B; p.N = N; p.C = C; p.H = heads; p.d = C / heads;
  const size_t lds = 2 * (size_t)p.d * ((N + 63) / 64) * sizeof(uint64_t);
  if (lds > 65536) return set_error(-2, "ssa_kv: (C/heads) * ceil(N/64) must be <= 4096 (token masks in LDS)");
  hipLaunchKernelGGL(ssa_kv_kernel, dim3((unsigned)(T * B * heads)), dim3(256), lds, stream, p);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_ssa_attend_neuron(int32_t T, int32_t B, int32_t N, int32_t C, int32_t heads, float scale,
                                             int32_t neuron, int32_t hard_reset, float tau, float v_threshold,
                                             float v_reset, const uint32_t* q_bits, const int32_t* kv,
                                             uint32_t* out_bits, hipStream_t stream) {
  if (const char* why = ssa_check(T, B, N, C, heads)) return set_error(-2, why);
  if (!q_bits || !kv || !out_bits) return set_error(-1, "ssa_attend_neuron: null pointer");
  if (const char* why = neuron_invalid(neuron, tau)) return set_error(-2, why);
  int e;
  if (!(scale > 0.f) || frexpf(scale, &e) != 0.5f)
    return set_error(-2, "ssa_attend_neuron: scale must be a power of two (exact attention arithmetic)");
  SsaParams p{};
  p.q = q_bits; p.kv = const_cast<int32_t*>(kv); p.out = reinterpret_cast<uint16_t*>(out_bits);
  p.T = T; p.B = B; p.N = N; p.C = C; p.H = heads; p.d = C / heads;
  p.xscale = scale * 0.5f;
  p.np = make_neuron_params(neuron, hard_reset, tau, v_threshold, v_reset);
  hipLaunchKernelGGL(ssa_attend_kernel, dim3((unsigned)(B * heads), (unsigned)((N + 63) / 64)), dim3(256), 0, stream,
                     p);
  return (int)hipGetLastError();
}
