// Spiking self-attention (Spikformer SSA, models/spikformer.py:103-130; the reference's
// TileLang matmul kernels, sengine/kernels/spikformer_kernels.py): per (t, b, head)
//     x = (Q K^T * scale) V,   then the attention neuron over T,
// with Q, K, V binary spikes (N tokens x d channels of the head).  Every product and
// partial sum is an integer (times scale, a power of two), exact in fp32 in any order, so
// this build evaluates x = Q (K^T V) * scale: K^T V is d x d, the work drops from
// N^2 d to N d^2 per head, and the result is bit-identical.
//
//   ssa_kv_kernel:     KV[t, b, h] = K^T V (int32 d x d).  A workgroup of 16 waves per
//                      (t*B + b, head pair), walking the tokens in chunks of 16 x 64: each
//                      wave turns 64 tokens' head slices into per-channel 64-token masks
//                      with a butterfly bit transpose across the wave (lane i ends with
//                      mask i), then threads add popcount(K_i & V_j) over the chunk's token
//                      masks to registers.
//   ssa_attend_kernel: X = Q KV on MFMA (v_mfma_f32_16x16x32_f16: A = KV^T as two exact
//                      fp16 pieces pre-scaled by a power of two -- the second only when
//                      some entry reaches 2048 --, B = Q expanded
//                      from bits, one fp32 accumulator), the neuron over T in
//                      registers, 16 output channels of a token assembled across lanes
//                      and stored as one u16.
#include <mutex>
#include <type_traits>

#include "common.h"
#include "epilogue.h"
#include "internal.h"

namespace sengine {

constexpr int kSsaMaxN = 8192;   // tokens (the attend kernel stages a workgroup's Q slices in LDS)
constexpr int kSsaMaxD = 64;
constexpr size_t kSsaMaxLds = 163840 - 256;  // attend kernel: KV pieces of every t and the staged Q slices (the
                                              // rest: the kernel's own workgroup reduction)

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

// 64 x 64 bit-matrix transpose across a wave: lane l holds row l (64 bits); afterwards lane c
// holds column c (bit l = row l's bit c).  Six butterfly stages swap the off-diagonal blocks of
// every 2d x 2d block: at stage d, a lane with bit d clear keeps the low d bits of each 2d-bit
// field and takes its partner's low d bits above them, a lane with bit d set keeps the high d
// bits and takes its partner's high d bits below them.  Branch-free: the partner's word rotated
// left by d (bit d clear) or right by d (set) -- one v_alignbit with a per-lane amount -- has
// the wanted bits where the lane does not keep its own, and the bits the rotation wraps around
// fall where it does; one bit-select merges them (as two selects of whole expressions, the
// stages compiled to divergent branches with the permute waits inside them).
__device__ __forceinline__ uint64_t transpose64(uint64_t x, int lane) {
  uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
  {  // d = 32: whole words
    const bool up = lane & 32;
    const uint32_t r = (uint32_t)__shfl_xor((int)(up ? lo : hi), 32, 64);
    lo = up ? r : lo;
    hi = up ? hi : r;
  }
  constexpr uint32_t kMask[5] = {0x0000ffffu, 0x00ff00ffu, 0x0f0f0f0fu, 0x33333333u, 0x55555555u};
#pragma unroll
  for (int st = 0; st < 5; ++st) {
    const int d = 16 >> st;
    const bool clear = (lane & d) == 0;
    const uint32_t keep = clear ? kMask[st] : ~kMask[st];  // the lane's own bits
    const uint32_t sh = clear ? 32u - d : (uint32_t)d;     // alignbit(x, x, sh): rotl by d or rotr by d
    const uint32_t plo = (uint32_t)__shfl_xor((int)lo, d, 64), phi = (uint32_t)__shfl_xor((int)hi, d, 64);
    lo = (lo & keep) | (__builtin_amdgcn_alignbit(plo, plo, sh) & ~keep);
    hi = (hi & keep) | (__builtin_amdgcn_alignbit(phi, phi, sh) & ~keep);
  }
  return ((uint64_t)hi << 32) | lo;
}

// A row slice of up to 256 bits (bit 0 = the slice's first bit) and the D bits at `bit`.
struct RowSlice {
  unsigned __int128 a, b;  // bits 0..127, 128..255
};
template <int D>
__device__ __forceinline__ uint64_t bits_at(const RowSlice& w, int bit) {
  uint64_t x;
  if (bit >= 128) {
    x = (uint64_t)(w.b >> (bit - 128));
  } else {
    x = (uint64_t)(w.a >> bit);
    if (bit + D > 128) x |= (uint64_t)(w.b << (128 - bit));
  }
  return D == 64 ? x : (x & ((1ull << D) - 1));
}

// Workgroup = (t*B + b, HP consecutive heads).  The tokens are walked in chunks of one 64-token
// group per wave: each wave loads its group's HP head slices (one contiguous run of the token
// row: HP heads share every cache line fetched), transposes each into per-channel token masks
// (the next chunk's rows are already in flight), and after a barrier every thread adds the
// popcounts of its (head, IB i, 16 j) item over a residue class of the chunk's groups to
// registers; the residues meet in LDS by integer atomics at the end (exact, order-free).
template <int D, int HP>
__global__ __launch_bounds__(64 * kSsaKvWaves) __attribute__((amdgpu_waves_per_eu(HP >= 4 ? 4 : 8))) void ssa_kv_kernel(SsaParams p) {
  constexpr int VS = D + 2;  // V mask j at j + j/32: reads of masks j0+u by the j0 = 0, 16, 32, 48 lane groups spread over bank pairs
  constexpr int NWS = (HP * D + 31) / 32 + (HP * D % 32 != 0 || HP == 1 ? 1 : 0);  // words of a row slice
  static_assert(NWS <= 8, "a row slice fits 256 bits");
  constexpr int JC = D / 16;
  constexpr int IB = 1;  // K channels per item (each V mask read feeds IB popcounts; 2 measured no faster)
  constexpr int ITEMS = HP * (D / IB) * JC;
  constexpr int R = kSsaKvWaves * 64 / ITEMS > 0 ? kSsaKvWaves * 64 / ITEMS : 1;
  // the chunk's K masks [HP][wave][D] and V masks [HP][wave][VS]; after the last chunk the same
  // memory holds the (head, i, j) sums
  constexpr int KM = HP * kSsaKvWaves * D, MW = KM + HP * kSsaKvWaves * VS, SW = (HP * D * D + 1) / 2;
  __shared__ uint64_t smem[MW > SW ? MW : SW];
  uint64_t* sKm = smem;       // [(e * kSsaKvWaves + g) * D + c]
  uint64_t* sVm = smem + KM;  // [(e * kSsaKvWaves + g) * VS + c]
  uint32_t* sum = reinterpret_cast<uint32_t*>(smem);  // [(e * D + i) * D + j]
  const int G = (p.N + 63) >> 6;
  const int nhb = p.H / HP;
  const int tb = blockIdx.x / nhb;
  const int h0 = (blockIdx.x - tb * nhb) * HP;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int words = p.C >> 5;
  const int w0 = (h0 * D) >> 5;                                  // first word of the slice
  const int sh = (HP * D) % 32 == 0 && HP > 1 ? 0 : ((h0 * D) & 31);  // its first bit within that word

  // this lane's token row slice (the HP heads' bits from word w0 on) of group g, k and v
  auto load = [&](int g, RowSlice& kw, RowSlice& vw) {
    const int n = (g << 6) + lane;
    const bool in = g < G && n < p.N;
    const size_t row = ((size_t)tb * p.N + (in ? n : 0)) * words + w0;
    uint32_t kx[NWS], vx[NWS];
    if constexpr (HP > 1) {  // the slice is whole words inside the row: one vector load each
      typedef uint32_t slice_t __attribute__((ext_vector_type(NWS), aligned(4)));
      const slice_t ka = *reinterpret_cast<const slice_t*>(p.k + row);
      const slice_t va = *reinterpret_cast<const slice_t*>(p.v + row);
#pragma unroll
      for (int u = 0; u < NWS; ++u) {
        kx[u] = in ? ka[u] : 0u;
        vx[u] = in ? va[u] : 0u;
      }
    } else {  // a head's bits may end in the row's last word
#pragma unroll
      for (int u = 0; u < NWS; ++u) {
        const bool ok = in && w0 + u < words;
        kx[u] = ok ? p.k[row + u] : 0u;
        vx[u] = ok ? p.v[row + u] : 0u;
      }
    }
    kw = vw = RowSlice{0, 0};
#pragma unroll
    for (int u = 0; u < NWS; ++u) {
      if (u < 4) {
        kw.a |= (unsigned __int128)kx[u] << (32 * u);
        vw.a |= (unsigned __int128)vx[u] << (32 * u);
      } else {
        kw.b |= (unsigned __int128)kx[u] << (32 * (u - 4));
        vw.b |= (unsigned __int128)vx[u] << (32 * (u - 4));
      }
    }
  };
  // this thread's item: head hh, channels i0 .. i0 + IB - 1 of K, channels j0 .. j0 + 15 of V, residue r
  const int r = (int)threadIdx.x / ITEMS;
  const int ij = (int)threadIdx.x - r * ITEMS;
  const int hh = ij / ((D / IB) * JC);
  const int i0 = (ij - hh * (D / IB) * JC) / JC * IB;
  const int j0 = (ij - hh * (D / IB) * JC - (i0 / IB) * JC) << 4;
  const bool active = r < R;
  uint32_t acc[IB][16];
#pragma unroll
  for (int a = 0; a < IB; ++a)
#pragma unroll
    for (int u = 0; u < 16; ++u) acc[a][u] = 0;

  RowSlice kn, vn;
  load(wave, kn, vn);
  for (int c0 = 0; c0 < G; c0 += kSsaKvWaves) {
    const RowSlice kw = kn, vw = vn;
    load(c0 + kSsaKvWaves + wave, kn, vn);
#pragma unroll
    for (int e = 0; e < HP; ++e) {
      // lane c: the token mask of channel c of head h0 + e (bit l = token l's bit c)
      const uint64_t km = transpose64(bits_at<D>(kw, e * D + sh), lane);
      const uint64_t vm = transpose64(bits_at<D>(vw, e * D + sh), lane);
      if (lane < D) {
        sKm[(e * kSsaKvWaves + wave) * D + lane] = km;
        sVm[(e * kSsaKvWaves + wave) * VS + lane + (lane >> 5)] = vm;
      }
    }
    __syncthreads();
    const int ng = min(kSsaKvWaves, G - c0);
    if (active) {
      for (int gg = r; gg < ng; gg += R) {
        uint64_t ki[IB];
#pragma unroll
        for (int a = 0; a < IB; ++a) ki[a] = sKm[(hh * kSsaKvWaves + gg) * D + i0 + a];
        const uint64_t* vj = sVm + (hh * kSsaKvWaves + gg) * VS + j0 + (j0 >> 5);  // j0 % 32 + 16 <= 32: one shift for all u
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const uint64_t vm = vj[u];
#pragma unroll
          for (int a = 0; a < IB; ++a) acc[a][u] += (uint32_t)__popcll(ki[a] & vm);
        }
      }
    }
    __syncthreads();
  }
  for (int idx = threadIdx.x; idx < HP * D * D; idx += blockDim.x) sum[idx] = 0u;
  __syncthreads();
  if (active) {
#pragma unroll
    for (int a = 0; a < IB; ++a)
#pragma unroll
      for (int u = 0; u < 16; ++u) atomicAdd(&sum[(hh * D + i0 + a) * D + j0 + u], acc[a][u]);
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < HP * D * D; idx += blockDim.x) {
    const int e = idx / (D * D);
    p.kv[((size_t)tb * p.H + h0 + e) * D * D + (idx - e * D * D)] = (int32_t)sum[idx];
  }
}

// Workgroup = (b, h, one of `splits` token ranges): KV of every t is staged once in LDS
// (fp16 pieces: the low 11 bits and the rest, exact, transposed to [j][i]); each wave then walks 16-token
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

  // stage: K^T V of every t as transposed fp16 pieces [t][piece][j][i].  The entries move as
  // 16-byte rows (4 consecutive j of one i), up to 8 per thread in flight before any is stored,
  // so the workgroup waits for a few round trips, not one per row.  Pieces are pre-scaled by
  // xscale (a power of two): the low 11 bits (x & 2047) and the rest (a multiple of 2048, at
  // most N) both stay exact in fp16, and both MFMAs accumulate x itself into one fp32
  // accumulator.  Entries below 2048 -- every entry unless some channel pair is set together in
  // 2048 tokens -- leave the high pieces zero, and a workgroup whose high pieces are all zero
  // skips their MFMAs (the same sums, exactly).
  _Float16* s = reinterpret_cast<_Float16*>(skv);
  constexpr int NV4 = T * D * D / 4;  // 16-byte rows
  constexpr int QB = 8;               // rows in flight per thread
  int high = 0;                       // any high piece of this thread's entries
  for (int base = threadIdx.x; base < NV4; base += 256 * QB) {
    int4 xv[QB];
#pragma unroll
    for (int r = 0; r < QB; ++r) {
      const int q4 = base + r * 256;
      if (q4 < NV4) {
        const int t = q4 / (D * D / 4);
        xv[r] = *reinterpret_cast<const int4*>(p.kv + ((size_t)(t * p.B + b) * p.H + h) * D * D +
                                                (size_t)(q4 - t * (D * D / 4)) * 4);
      }
    }
#pragma unroll
    for (int r = 0; r < QB; ++r) {
      const int q4 = base + r * 256;
      if (q4 < NV4) {
        const int t = q4 / (D * D / 4), rem = q4 - t * (D * D / 4);
        const int i = rem / (D / 4), j0 = (rem - i * (D / 4)) * 4;
        const int xs[4] = {xv[r].x, xv[r].y, xv[r].z, xv[r].w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          s[((size_t)(t * 2 + 0) * D + j0 + u) * kSsaRow + i] = (_Float16)((float)(xs[u] & 2047) * p.xscale);
          s[((size_t)(t * 2 + 1) * D + j0 + u) * kSsaRow + i] = (_Float16)((float)(xs[u] & ~2047) * p.xscale);
          high |= xs[u] & ~2047;
        }
      }
    }
  }
  if (D < 64) {  // rows i = D .. 63 of the last k step read as zero
    for (int idx = threadIdx.x; idx < T * 2 * D * (64 - D); idx += 256) {
      const int row = idx / (64 - D);
      s[(size_t)row * kSsaRow + D + (idx - row * (64 - D))] = (_Float16)0.f;
    }
  }
  const bool big = __syncthreads_or(high != 0);  // some high piece is nonzero (workgroup-uniform)

  const int tiles = (p.N + 15) >> 4;
  const int per = (tiles + splits - 1) / splits;
  const int tile0 = split * per;
  const int tile_end = min(tiles, tile0 + per);
  // Every Q slice of the workgroup's tokens is staged in LDS before the first output store:
  // the vector-memory counter also counts stores, so a load waited for after stores would
  // wait for those stores too.
  uint64_t* sq = reinterpret_cast<uint64_t*>(skv + (size_t)T * 2 * D * RV);  // [t][token]
  const int ntok = (tile_end - tile0) * 16;
  for (int base = threadIdx.x; base < T * ntok; base += 256 * QB) {  // QB slices in flight per thread
    uint64_t qs[QB];
#pragma unroll
    for (int r = 0; r < QB; ++r) {
      const int idx = base + r * 256;
      const int t = idx / ntok, n = tile0 * 16 + idx - t * ntok;
      qs[r] = idx < T * ntok && n < p.N
                  ? head_slice(p.q + ((size_t)(t * p.B + b) * p.N + n) * words, words, h * D, D)
                  : 0ull;
    }
#pragma unroll
    for (int r = 0; r < QB; ++r)
      if (base + r * 256 < T * ntok) sq[base + r * 256] = qs[r];
  }
  __syncthreads();
  // per-step strides, hoisted out of the tile loop (the loop otherwise recomputes the 32- and
  // 64-bit products for every step, on the quarter-rate integer multiplier)
  const size_t out_tstride = (size_t)p.B * p.N * p.C / 16;  // u16 words per timestep
  uint16_t* const out_bh = p.out + ((size_t)b * p.N * p.C + h * D) / 16;
  for (int tile = tile0 + wave; tile < tile_end; tile += 4) {
    uint64_t qcur[T];
    const uint64_t* sqt = sq + (tile - tile0) * 16 + c;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      qcur[t] = *sqt;
      sqt += ntok;
    }
    const int n = tile * 16 + c;  // this lane's token (MFMA column)
    const bool nvalid = n < p.N;
    uint16_t* o = out_bh + (size_t)n * (p.C / 16);
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
      auto mma = [&](auto with_high) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const half8_t bq = expand_bits8((uint32_t)(qcur[t] >> (32 * ks + 8 * g)) & 0xffu);
#pragma unroll
          for (int jt = 0; jt < JT; ++jt) {
            const half8_t a0 = st[(size_t)(jt * 16 + c) * RV + ks * 4 + g];
            acc[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bq, acc[jt], 0, 0, 0);
            if constexpr (decltype(with_high)::value) {
              const half8_t a1 = st[(size_t)(D + jt * 16 + c) * RV + ks * 4 + g];
              acc[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bq, acc[jt], 0, 0, 0);
            }
          }
        }
      };
      if (big) mma(std::true_type{});
      else mma(std::false_type{});
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
#pragma unroll
        for (int jt = 0; jt < JT; ++jt) o[jt] = (uint16_t)word[jt];
      }
      o += out_tstride;
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
  int hp;  // heads per workgroup
};

int kv_setup(int32_t T, int32_t B, int32_t N, int32_t C, int32_t heads, const uint32_t* k_bits,
             const uint32_t* v_bits, int32_t* kv, KvLaunch& L) {
  if (const char* why = ssa_check(T, B, N, C, heads)) return set_error(-2, why);
  if (!k_bits || !v_bits || !kv) return set_error(-1, "ssa_kv: null pointer");
  SsaParams& p = L.p;
  p = SsaParams{};
  p.k = k_bits; p.v = v_bits; p.kv = kv;
  p.T = T; p.B = B; p.N = N; p.C = C; p.H = heads; p.d = C / heads;
  // heads per workgroup: the heads of one workgroup share the cache lines of their token rows
  // (a line request per lane and row serves all of them); four while the chunk's masks fit LDS
  L.hp = heads % 4 == 0 && p.d <= 48 ? 4 : heads % 2 == 0 ? 2 : 1;
  return 0;
}

template <int HP>
int kv_launch_hp(const SsaParams& p, dim3 grid, hipStream_t stream) {
  const dim3 block(64 * kSsaKvWaves);
  switch (p.d) {
    case 16: hipLaunchKernelGGL((ssa_kv_kernel<16, HP>), grid, block, 0, stream, p); break;
    case 32: hipLaunchKernelGGL((ssa_kv_kernel<32, HP>), grid, block, 0, stream, p); break;
    case 48: hipLaunchKernelGGL((ssa_kv_kernel<48, HP>), grid, block, 0, stream, p); break;
    default:
      if constexpr (HP == 4) return set_error(-2, "ssa_kv: four heads per workgroup need head dim <= 48");
      else hipLaunchKernelGGL((ssa_kv_kernel<64, HP>), grid, block, 0, stream, p);
  }
  return (int)hipGetLastError();
}

int kv_launch(const KvLaunch& L, hipStream_t stream) {
  const SsaParams& p = L.p;
  const dim3 grid((unsigned)(p.T * p.B * p.H / L.hp));
  if (L.hp == 4) return kv_launch_hp<4>(p, grid, stream);
  if (L.hp == 2) return kv_launch_hp<2>(p, grid, stream);
  return kv_launch_hp<1>(p, grid, stream);
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
  // token ranges per (b, head): about 1024 workgroups (four rounds of one per CU), at least 4 tiles each
  const int tiles = (N + 15) / 16;
  L.splits = std::max(1, std::min((tiles + 3) / 4, (1024 + B * heads - 1) / (B * heads)));
  const int per = (tiles + L.splits - 1) / L.splits;
  L.lds = (size_t)T * 2 * p.d * kSsaRow * sizeof(_Float16) + (size_t)T * per * 16 * sizeof(uint64_t);
  if (L.lds > kSsaMaxLds)
    return set_error(-2, "ssa_attend_neuron: T * (C/heads) and the token range too large for LDS");
  // fast path: LIF with an exact power-of-two 1/tau and decay, hard reset (the reference's attn_lif)
  const bool fast = epilogue_mode(p.np, false) == EPI_LIF_HARD;
  L.fn = p.d == 16 ? attend_fn<16>(T, fast) : p.d == 32 ? attend_fn<32>(T, fast)
                                             : p.d == 48 ? attend_fn<48>(T, fast) : attend_fn<64>(T, fast);
  if (fast) p.xscale *= p.np.rtau;  // exact: both powers of two
  // the K^T V entries (integers <= N) go to fp16 as (x & 2047) * xscale and (x & ~2047) *
  // xscale: exact only while the larger stays finite and the smaller's unit is representable
  if ((double)N * p.xscale > 65504.0 || p.xscale < 0x1p-24f)
    return set_error(-2, "ssa_attend_neuron: scale out of range for exact fp16 attention pieces (needs "
                         "N * scale / 2 <= 65504 and scale / 2 >= 2^-24, times 1/tau for LIF)");
  return 0;
}

int attend_launch(AttendLaunch& L, hipStream_t stream) {
  if (L.lds > 65536) {  // opt in to more than 64 KB of dynamic LDS (a host-side attribute)
    const hipError_t e2 = hipFuncSetAttribute(L.fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)L.lds);
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
