// Spiking self-attention (Spikformer SSA, models/spikformer.py:103-130; the reference's
// TileLang matmul kernels, sengine/kernels/spikformer_kernels.py): per (t, b, head)
//     x = (Q K^T * scale) V,   then the attention neuron over T,
// with Q, K, V binary spikes (N tokens x d channels of the head).  Every product and
// partial sum is an integer (times scale, a power of two), exact in fp32 in any order, so
// this build evaluates x = Q (K^T V) * scale: K^T V is d x d, the work drops from
// N^2 d to N d^2 per head, and the result is bit-identical.
//
//   ssa_kv_kernel:     KV[t, b, h] = K^T V (int32 d x d).  A workgroup of 16 waves per
//                      (t*B + b, h): each wave turns 64 tokens' head slices into
//                      per-channel 64-token masks with ballots (bit transposition; lane i
//                      collects mask i, one wave-wide LDS store per group), then threads
//                      sum popcount(K_i & V_j) over the token masks.
//   ssa_attend_kernel: X = Q KV on MFMA (v_mfma_f32_16x16x32_f16: A = KV^T as two exact
//                      6-bit fp16 pieces pre-scaled by a power of two, B = Q expanded
//                      from bits, one fp32 accumulator), the neuron over T in
//                      registers, 16 output channels of a token assembled across lanes
//                      and stored as one u16.
#include <mutex>

#include "common.h"
#include "epilogue.h"
#include "internal.h"

namespace sengine {

constexpr int kSsaMaxN = 8192;   // tokens (the KV kernel keeps 2 x d x N/64 token masks in LDS)
constexpr int kSsaMaxD = 64;
constexpr size_t kSsaMaxLds = 163840;  // attend kernel: KV pieces of every t and the staged Q slices

struct SsaParams {
  const uint32_t* q;
  const uint32_t* k;
  const uint32_t* v;
  int32_t* kv;     // (T*B, H, d, d)
  uint16_t* out;   // spike bits (T*B, N, C) viewed as u16 words
  int T, B, N, C, H, d;
  float xscale;    // scale / 2 (the MFMA sees spikes as 2.0), times 1/tau on the fast path
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

constexpr int kSsaKvWaves = 16;

template <int D>
__global__ __launch_bounds__(64 * kSsaKvWaves) void ssa_kv_kernel(SsaParams p) {
  // K masks [G][D], then V masks [G][VS] (mask j at j + j/32: a read of masks j0+u by lane
  // groups j0 = 0, 16, 32, 48 hits four different bank pairs), then the KV sums
  extern __shared__ uint64_t masks[];
  constexpr int VS = D + 2;
  const int G = (p.N + 63) >> 6;
  uint64_t* Km = masks;
  uint64_t* Vm = masks + (size_t)D * G;
  uint32_t* sum = reinterpret_cast<uint32_t*>(masks + (size_t)(D + VS) * G);  // [D][D]
  for (int idx = threadIdx.x; idx < D * D; idx += blockDim.x) sum[idx] = 0u;
  const int tb = blockIdx.x / p.H;
  const int h = blockIdx.x - tb * p.H;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int words = p.C >> 5;
  // this lane's token slices, loaded one token group ahead of the ballots
  auto load = [&](int g, uint64_t& ks, uint64_t& vs) {
    const int n = (g << 6) + lane;
    ks = vs = 0;
    if (g < G && n < p.N) {
      const size_t row = ((size_t)tb * p.N + n) * words;
      ks = head_slice(p.k + row, words, h * D, D);
      vs = head_slice(p.v + row, words, h * D, D);
    }
  };
  uint64_t ksn, vsn;
  load(wave, ksn, vsn);
  for (int g = wave; g < G; g += kSsaKvWaves) {
    const uint32_t k0 = (uint32_t)ksn, k1 = (uint32_t)(ksn >> 32);
    const uint32_t v0 = (uint32_t)vsn, v1 = (uint32_t)(vsn >> 32);
    load(g + kSsaKvWaves, ksn, vsn);
    // compile-time bit masks: one test and one ballot per bit; lane i keeps mask i, so the
    // group's masks go to LDS as two wave-wide stores instead of 2*D single-lane ones
    int km0 = 0, km1 = 0, vm0 = 0, vm1 = 0;  // lane i: mask i (low, high word)
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const uint64_t mk = __ballot(((i < 32 ? k0 : k1) >> (i & 31)) & 1u);
      const uint64_t mv = __ballot(((i < 32 ? v0 : v1) >> (i & 31)) & 1u);
      // the ballot's SGPRs come from a VALU compare: wait states before v_writelane reads
      // them (the compiler's hazard recognizer does not look inside inline asm)
      asm("s_nop 4\n\tv_writelane_b32 %0, %1, %2" : "+v"(km0) : "s"((uint32_t)mk), "i"(i));
      asm("v_writelane_b32 %0, %1, %2" : "+v"(km1) : "s"((uint32_t)(mk >> 32)), "i"(i));
      asm("s_nop 4\n\tv_writelane_b32 %0, %1, %2" : "+v"(vm0) : "s"((uint32_t)mv), "i"(i));
      asm("v_writelane_b32 %0, %1, %2" : "+v"(vm1) : "s"((uint32_t)(mv >> 32)), "i"(i));
    }
    if (lane < D) {
      Km[(size_t)g * D + lane] = ((uint64_t)(uint32_t)km1 << 32) | (uint32_t)km0;
      Vm[(size_t)g * VS + lane + (lane >> 5)] = ((uint64_t)(uint32_t)vm1 << 32) | (uint32_t)vm0;
    }
  }
  __syncthreads();
  // work item = (i, 16 consecutive j, token-group residue r): K_i masks read once per
  // token group; the residues' partial counts meet in LDS by integer atomics (exact, order-free)
  constexpr int JC = D / 16;
  constexpr int R = kSsaKvWaves * 64 / (D * JC) > 0 ? kSsaKvWaves * 64 / (D * JC) : 1;
  for (int item = threadIdx.x; item < D * JC * R; item += blockDim.x) {
    const int r = item / (D * JC);
    const int ij = item - r * (D * JC);
    const int i = ij / JC;
    const int j0 = (ij - i * JC) << 4;
    uint32_t acc[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) acc[u] = 0;
    for (int g = r; g < G; g += R) {
      const uint64_t ki = Km[(size_t)g * D + i];
      const uint64_t* vj = Vm + (size_t)g * VS + j0 + (j0 >> 5);  // j0 % 32 + 16 <= 32: one shift for all u
#pragma unroll
      for (int u = 0; u < 16; ++u) acc[u] += (uint32_t)__popcll(ki & vj[u]);
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) atomicAdd(&sum[i * D + j0 + u], acc[u]);
  }
  __syncthreads();
  int32_t* kv = p.kv + (size_t)blockIdx.x * D * D;
  for (int idx = threadIdx.x; idx < D * D; idx += blockDim.x) kv[idx] = (int32_t)sum[idx];
}

// Workgroup = (b, h, one of `splits` token ranges): KV of every t is staged once in LDS
// (fp16 hi/lo 6-bit pieces, exact, transposed to [j][i]); each wave then walks 16-token
// tiles, t inner, membrane in registers.  MFMA roles: D[j][token] = sum_i KV^T[j][i] *
// Q^T[i][token].
constexpr int kSsaRow = 72;  // fp16 per staged KV row: i padded to 64 plus 8 (bank spread)

template <int D, int T, int MODE>
__global__ __launch_bounds__(256) void ssa_attend_kernel(SsaParams p, int splits) {
  extern __shared__ half8_t skv[];  // [t][piece][j][kSsaRow / 8]
  constexpr int JT = D / 16;        // j tiles of 16
  constexpr int KS = (D + 31) / 32; // k steps of 32 channels
  constexpr int RV = kSsaRow / 8;   // half8 per row
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int bh = blockIdx.x / splits;
  const int split = blockIdx.x - bh * splits;
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int words = p.C >> 5;
  const bool fold = p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2;

  // stage: a wave per (t, i) row, lanes over j (coalesced reads), transposed fp16 pieces
  _Float16* s = reinterpret_cast<_Float16*>(skv);
  for (int ti = wave; ti < T * 64; ti += 4) {
    const int t = ti >> 6, i = ti & 63;
    if (lane < D) {
      // pieces pre-scaled by xscale (a power of two): lo * xs and hi * 64 * xs stay exact in
      // fp16, and both MFMAs accumulate x itself into one fp32 accumulator
      const int32_t x = i < D ? p.kv[((size_t)(t * p.B + b) * p.H + h) * D * D + i * D + lane] : 0;
      s[((size_t)(t * 2 + 0) * D + lane) * kSsaRow + i] = (_Float16)((float)(x & 63) * p.xscale);
      s[((size_t)(t * 2 + 1) * D + lane) * kSsaRow + i] = (_Float16)((float)((x >> 6) << 6) * p.xscale);
    }
  }
  __syncthreads();

  const int tiles = (p.N + 15) >> 4;
  const int per = (tiles + splits - 1) / splits;
  const int tile0 = split * per;
  const int tile_end = min(tiles, tile0 + per);
  // Every Q slice of the workgroup's tokens is staged in LDS before the first output store:
  // the vector-memory counter also counts stores, so a load waited for after stores would
  // wait for those stores too.
  uint64_t* sq = reinterpret_cast<uint64_t*>(skv + (size_t)T * 2 * D * RV);  // [t][token]
  const int ntok = (tile_end - tile0) * 16;
  for (int idx = threadIdx.x; idx < T * ntok; idx += blockDim.x) {
    const int t = idx / ntok, k = idx - (idx / ntok) * ntok;
    const int n = tile0 * 16 + k;
    sq[idx] = n < p.N ? head_slice(p.q + ((size_t)(t * p.B + b) * p.N + n) * words, words, h * D, D) : 0ull;
  }
  __syncthreads();
  for (int tile = tile0 + wave; tile < tile_end; tile += 4) {
    uint64_t qcur[T];
#pragma unroll
    for (int t = 0; t < T; ++t) qcur[t] = sq[t * ntok + (tile - tile0) * 16 + c];
    const int n = tile * 16 + c;  // this lane's token (MFMA column)
    const bool nvalid = n < p.N;
    float v[JT][4];  // membrane per (j tile, row e)
#pragma unroll
    for (int jt = 0; jt < JT; ++jt)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[jt][e] = 0.f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const half8_t* st = skv + (size_t)t * 2 * D * RV;
      float4_t acc[JT];
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) acc[jt] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const half8_t bq = expand_bits8((uint32_t)(qcur[t] >> (32 * ks + 8 * g)) & 0xffu);
#pragma unroll
        for (int jt = 0; jt < JT; ++jt) {
          const half8_t a0 = st[(size_t)(jt * 16 + c) * RV + ks * 4 + g];
          const half8_t a1 = st[(size_t)(D + jt * 16 + c) * RV + ks * 4 + g];
          acc[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bq, acc[jt], 0, 0, 0);
          acc[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bq, acc[jt], 0, 0, 0);
        }
      }
      // neuron on x[token][j = 16 jt + 4 g + e]; 16 spikes of a token gathered from 4 lanes
      uint32_t word[JT];
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        uint32_t nib = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = acc[jt][e];  // the attention output (times 1/tau on the fast path), exact
          if (MODE == EPI_LIF_HARD) {
            const float hh = __builtin_fmaf(v[jt][e], p.np.decay, x);  // v*decay exact: one rounding
            const bool spike = hh >= p.np.vth;
            v[jt][e] = spike ? p.np.vreset : hh;
            nib |= (uint32_t)spike << e;
          } else {
            const float xf = fold ? x * p.np.rtau : x;
            const float hh = neuron_charge(p.np, v[jt][e], xf);
            const bool spike = hh >= p.np.vth;
            v[jt][e] = neuron_reset(p.np, hh, spike);
            nib |= (uint32_t)spike << e;
          }
        }
        const uint32_t n1 = __shfl(nib, c + 16, 64), n2 = __shfl(nib, c + 32, 64), n3 = __shfl(nib, c + 48, 64);
        word[jt] = nib | (n1 << 4) | (n2 << 8) | (n3 << 12);
      }
      if (g == 0 && nvalid) {
        uint16_t* o = p.out + (((size_t)(t * p.B + b) * p.N + n) * p.C + h * D) / 16;
#pragma unroll
        for (int jt = 0; jt < JT; ++jt) o[jt] = (uint16_t)word[jt];
      }
    }
  }
}

template <int D, int T>
static void* attend_fn_t(bool fast) {
  return fast ? reinterpret_cast<void*>(&ssa_attend_kernel<D, T, EPI_LIF_HARD>)
              : reinterpret_cast<void*>(&ssa_attend_kernel<D, T, EPI_GENERIC>);
}

template <int D>
static void* attend_fn(int T, bool fast) {
  switch (T) {
    case 1: return attend_fn_t<D, 1>(fast);
    case 2: return attend_fn_t<D, 2>(fast);
    case 4: return attend_fn_t<D, 4>(fast);
    default: return attend_fn_t<D, 8>(fast);
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

namespace {

struct KvLaunch {
  SsaParams p;
  size_t lds;
};

int kv_setup(int32_t T, int32_t B, int32_t N, int32_t C, int32_t heads, const uint32_t* k_bits,
             const uint32_t* v_bits, int32_t* kv, KvLaunch& L) {
  if (const char* why = ssa_check(T, B, N, C, heads)) return set_error(-2, why);
  if (!k_bits || !v_bits || !kv) return set_error(-1, "ssa_kv: null pointer");
  SsaParams& p = L.p;
  p = SsaParams{};
  p.k = k_bits; p.v = v_bits; p.kv = kv;
  p.T = T; p.B = B; p.N = N; p.C = C; p.H = heads; p.d = C / heads;
  L.lds = (2 * (size_t)p.d + 2) * ((N + 63) / 64) * sizeof(uint64_t) + (size_t)p.d * p.d * sizeof(uint32_t);
  if (L.lds > 65536) return set_error(-2, "ssa_kv: (C/heads) * ceil(N/64) too large for the token masks in LDS");
  return 0;
}

int kv_launch(const KvLaunch& L, hipStream_t stream) {
  const SsaParams& p = L.p;
  const dim3 grid((unsigned)(p.T * p.B * p.H)), block(64 * kSsaKvWaves);
  switch (p.d) {
    case 16: hipLaunchKernelGGL(ssa_kv_kernel<16>, grid, block, L.lds, stream, p); break;
    case 32: hipLaunchKernelGGL(ssa_kv_kernel<32>, grid, block, L.lds, stream, p); break;
    case 48: hipLaunchKernelGGL(ssa_kv_kernel<48>, grid, block, L.lds, stream, p); break;
    default: hipLaunchKernelGGL(ssa_kv_kernel<64>, grid, block, L.lds, stream, p); break;
  }
  return (int)hipGetLastError();
}

struct AttendLaunch {
  SsaParams p;
  void* fn;
  size_t lds;
  int splits;
};

int attend_setup(int32_t T, int32_t B, int32_t N, int32_t C, int32_t heads, float scale, int32_t neuron,
                 int32_t hard_reset, float tau, float v_threshold, float v_reset, const uint32_t* q_bits,
                 const int32_t* kv, uint32_t* out_bits, AttendLaunch& L) {
  if (const char* why = ssa_check(T, B, N, C, heads)) return set_error(-2, why);
  if (!q_bits || !kv || !out_bits) return set_error(-1, "ssa_attend_neuron: null pointer");
  if (const char* why = neuron_invalid(neuron, tau)) return set_error(-2, why);
  if (T != 1 && T != 2 && T != 4 && T != 8) return set_error(-2, "ssa_attend_neuron: T must be 1, 2, 4 or 8");
  int e;
  if (!(scale > 0.f) || frexpf(scale, &e) != 0.5f)
    return set_error(-2, "ssa_attend_neuron: scale must be a power of two (exact attention arithmetic)");
  SsaParams& p = L.p;
  p = SsaParams{};
  p.q = q_bits; p.kv = const_cast<int32_t*>(kv); p.out = reinterpret_cast<uint16_t*>(out_bits);
  p.T = T; p.B = B; p.N = N; p.C = C; p.H = heads; p.d = C / heads;
  p.xscale = scale * 0.5f;
  p.np = make_neuron_params(neuron, hard_reset, tau, v_threshold, v_reset);
  // token ranges per (b, head): enough workgroups for every CU several times over
  const int tiles = (N + 15) / 16;
  L.splits = std::max(1, std::min((tiles + 3) / 4, (2048 + B * heads - 1) / (B * heads)));
  const int per = (tiles + L.splits - 1) / L.splits;
  L.lds = (size_t)T * 2 * p.d * kSsaRow * sizeof(_Float16) + (size_t)T * per * 16 * sizeof(uint64_t);
  if (L.lds > kSsaMaxLds)
    return set_error(-2, "ssa_attend_neuron: T * (C/heads) and the token range too large for LDS");
  // fast path: LIF with an exact power-of-two 1/tau and decay, hard reset (the reference's attn_lif)
  const bool fast = epilogue_mode(p.np, false) == EPI_LIF_HARD;
  L.fn = p.d == 16 ? attend_fn<16>(T, fast) : p.d == 32 ? attend_fn<32>(T, fast)
                                             : p.d == 48 ? attend_fn<48>(T, fast) : attend_fn<64>(T, fast);
  if (fast) p.xscale *= p.np.rtau;  // exact: both powers of two
  // the K^T V entries (integers <= N) go to fp16 as (x & 63) * xscale and ((x >> 6) << 6) *
  // xscale: exact only while the larger stays finite and the smaller's unit is representable
  if ((double)N * p.xscale > 65504.0 || p.xscale < 0x1p-24f)
    return set_error(-2, "ssa_attend_neuron: scale out of range for exact fp16 attention pieces (needs "
                         "N * scale / 2 <= 65504 and scale / 2 >= 2^-24, times 1/tau for LIF)");
  return 0;
}

int attend_launch(AttendLaunch& L, hipStream_t stream) {
  if (L.lds > 65536) {  // opt in to more than 64 KB of dynamic LDS (a host-side attribute)
    const hipError_t e2 = hipFuncSetAttribute(L.fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kSsaMaxLds);
    if (e2 != hipSuccess) return (int)e2;
  }
  void* args[] = {&L.p, &L.splits};
  return (int)hipLaunchKernel(L.fn, dim3((unsigned)(L.p.B * L.p.H * L.splits)), dim3(256), args, L.lds, stream);
}

// Allocation-free attention: K^T V in a file-scope device array instead of a caller workspace.
// Each GPU holds its own copy; its address is taken once per device (host code never passes
// the array's name itself, which on the host is only a stand-in for the symbol).
constexpr size_t kSsaScratchInts = size_t(1) << 22;  // 16 MiB: T*B*heads*d*d int32 at most
static __device__ __align__(256) int32_t scratch[kSsaScratchInts];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
int32_t* g_scratch[kMaxDevices] = {};

int scratch_for_current_device(int32_t** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return set_error(-2, "ssa_attention_noalloc: device index beyond 64");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!ptr) return set_error(-1, "ssa_attention_noalloc: no address for the scratch array");
    g_scratch[dev] = static_cast<int32_t*>(ptr);
  }
  *out = g_scratch[dev];
  return 0;
}

}  // namespace
}  // namespace sengine

using namespace sengine;

extern "C" int sengine_amd_ssa_kv(int32_t T, int32_t B, int32_t N, int32_t C, int32_t heads, const uint32_t* k_bits,
                                  const uint32_t* v_bits, int32_t* kv, hipStream_t stream) {
  KvLaunch L;
  const int rc = kv_setup(T, B, N, C, heads, k_bits, v_bits, kv, L);
  return rc ? rc : kv_launch(L, stream);
}

extern "C" int sengine_amd_ssa_attend_neuron(int32_t T, int32_t B, int32_t N, int32_t C, int32_t heads, float scale,
                                             int32_t neuron, int32_t hard_reset, float tau, float v_threshold,
                                             float v_reset, const uint32_t* q_bits, const int32_t* kv,
                                             uint32_t* out_bits, hipStream_t stream) {
  AttendLaunch L;
  const int rc = attend_setup(T, B, N, C, heads, scale, neuron, hard_reset, tau, v_threshold, v_reset, q_bits, kv,
                              out_bits, L);
  return rc ? rc : attend_launch(L, stream);
}

extern "C" int sengine_amd_ssa_attention_noalloc(int32_t T, int32_t B, int32_t N, int32_t C, int32_t heads,
                                                 float scale, int32_t neuron, int32_t hard_reset, float tau,
                                                 float v_threshold, float v_reset, const uint32_t* q_bits,
                                                 const uint32_t* k_bits, const uint32_t* v_bits, uint32_t* out_bits,
                                                 hipStream_t stream) {
  if (const char* why = ssa_check(T, B, N, C, heads)) return set_error(-2, why);
  const size_t d = (size_t)(C / heads);
  if ((size_t)T * B * heads * d * d > kSsaScratchInts)
    return set_error(-2, "ssa_attention_noalloc: T * B * heads * (C/heads)^2 exceeds the 4,194,304-entry scratch");
  int32_t* kv = nullptr;
  int rc = scratch_for_current_device(&kv);
  if (rc) return rc;
  // every argument is checked before anything is launched
  KvLaunch K;
  if ((rc = kv_setup(T, B, N, C, heads, k_bits, v_bits, kv, K))) return rc;
  AttendLaunch A;
  if ((rc = attend_setup(T, B, N, C, heads, scale, neuron, hard_reset, tau, v_threshold, v_reset, q_bits, kv,
                         out_bits, A)))
    return rc;
  // the K^T V kernel writes every entry the attend kernel reads: nothing to clear
  if ((rc = kv_launch(K, stream))) return rc;
  return attend_launch(A, stream);
}
