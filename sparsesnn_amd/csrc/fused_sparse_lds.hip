// Fused 2:4-sparse Conv + BN + multi-step LIF/IF for spike-bit inputs (gfx950 fast path).
//
// Same operator and GEMM view as fused_sparse.hip (see there), restructured for the
// MI355X's measured limits: a v_smfmac_f32_16x16x64_f16 issues every ~18 cycles per
// SIMD, each extra VALU op per SMFMAC costs ~3.5 cycles, LDS delivers ~128 B/clk/CU.
//
//  * Workgroup = 4 waves = 64 output channels x 64*PT positions (flattened (b, oh, ow),
//    the reference's M_per_t order).  Wave w owns 16*PT positions, all 64 channels and
//    all T timesteps: T*4*PT accumulator tiles in registers.
//  * The reduction runs over chunks q = (kh, kw, 64 input channels), advanced with
//    counters (no integer division in the loop).  Each chunk is staged into LDS by the
//    whole workgroup, double-buffered so the global loads of chunk q+1 are in flight
//    while chunk q is multiplied (a two-chunk-deep prefetch measured slower: the second
//    register set costs occupancy):
//      - the 4 weight fragments (A operands, 1 KB each) and their 2-bit metadata;
//      - one 64-bit spike word per (timestep, position): the tap-shifted input pixel's
//        64 channel bits (zero outside the image: the conv's zero padding), bytes
//        interleaved [b0 b4 b1 b5 b2 b6 b3 b7] so lane group g reads its 16 bits
//        (channels 8g..8g+7 and 32+8g..32+8g+7, the SMFMAC B layout) as one u16.
//  * Per chunk a wave reads its A operands once and reuses them for T*PT B fragments;
//    each B fragment (16 bits -> 16 fp16 values, 16 VALU ops) feeds 4 SMFMACs.
//  * Epilogue (epilogue.h): folded BN + T-step neuron in registers, 16 spike bits per
//    lane per timestep stored as one u16 (NHWC spike bits).
#include "common.h"
#include "epilogue.h"
#include "internal.h"

#include <stdlib.h>

namespace sengine {

struct LdsParams {
  const uint8_t* in;
  const u32x4_t* wvals;
  const uint32_t* wmeta;
  float* state;
  const float* scale;
  const float* bias;
  uint8_t* out;
  float* h_trace;
  float* x_trace;
  int B, C, H, W, F, KW, SH, SW, PH, PW, DH, DW, OH, OW;
  int M, nq;
  int64_t in_t_bytes;  // bytes of one timestep of input spike bits
  NeuronParams np;
  float enc_scale;
};

__device__ __forceinline__ uint2 interleave_bytes(uint2 w) {
  // [b0 b1 b2 b3 | b4 b5 b6 b7] -> [b0 b4 b1 b5 | b2 b6 b3 b7]
  return uint2{__builtin_amdgcn_perm(w.y, w.x, 0x05010400u), __builtin_amdgcn_perm(w.y, w.x, 0x07030602u)};
}

// Registers holding one chunk's staged data between its global load and its LDS store.
template <int NW, int PL>
struct StageRegs {
  uint2 bw[NW];
  u32x4_t aw[PL];
  uint32_t mw;
};

// Workgroup order: hardware dispatches consecutive workgroup ids round-robin over the 8
// XCDs (separate L2s).  Remap so each XCD receives a contiguous run of position tiles,
// keeping the input rows shared by neighbouring tiles in one L2.
__device__ __forceinline__ int xcd_tile(int id, int n) {
  const int per = n >> 3;                 // full tiles per XCD
  if (id >= per * 8) return id;           // ragged tail keeps its id
  return (id & 7) * per + (id >> 3);
}

template <int T, int PT, int PL, int OUT_ENC, int MODE>
__global__ __launch_bounds__(256) void fused_sparse_lds_kernel(LdsParams p) {
  constexpr int NPOS = 64 * PT;                  // positions per workgroup
  constexpr int TSTEP = 256 / NPOS;              // timesteps covered by one pass of 256 threads
  constexpr int NW = (T + TSTEP - 1) / TSTEP;    // spike words staged per thread per chunk
  __shared__ uint2 sB[2][T][NPOS];
  __shared__ u32x4_t sA[2][PL][256];
  __shared__ uint32_t sM[2][256];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int col = lane & 15;
  const int G = blockIdx.y;
  const int m0 = xcd_tile(blockIdx.x, gridDim.x) * NPOS;

  // ---- staging identity: one position, timesteps st0, st0+TSTEP, ...
  const int spos = tid % NPOS;
  const int st0 = tid / NPOS;
  const int sm = m0 + spos;
  const bool svalid = sm < p.M;
  int sb = 0, soh = 0, sow = 0;
  if (svalid) {
    const int ohw = p.OH * p.OW;
    sb = sm / ohw;
    const int r = sm - sb * ohw;
    soh = r / p.OW;
    sow = r - soh * p.OW;
  }
  const int ih0 = soh * p.SH - p.PH;
  const int iw0 = sow * p.SW - p.PW;
  const int cbytes = p.C >> 3;
  const u32x4_t* wv = p.wvals + (size_t)G * p.nq * PL * 256 + tid;
  const uint32_t* wm = p.wmeta + (size_t)G * p.nq * 256 + tid;

  // chunk counters of the next chunk to load: q = (kr, ks, c0), uniform in the workgroup
  int lq = 0, kr = 0, ks = 0, c0 = 0;
  auto load_next = [&](StageRegs<NW, PL>& R) {
    if (lq < p.nq) {
      const int ih = ih0 + kr * p.DH;
      const int iw = iw0 + ks * p.DW;
      const bool ok = svalid && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W;
      const int64_t base = (((int64_t)sb * p.H + ih) * p.W + iw) * cbytes + (c0 >> 3);
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        const int t = st0 + k * TSTEP;
        R.bw[k] = uint2{0u, 0u};
        if (ok && t < T) R.bw[k] = *reinterpret_cast<const uint2*>(p.in + base + t * p.in_t_bytes);
      }
#pragma unroll
      for (int pl = 0; pl < PL; ++pl) R.aw[pl] = wv[((size_t)lq * PL + pl) * 256];
      R.mw = wm[(size_t)lq * 256];
      c0 += 64;
      if (c0 == p.C) {
        c0 = 0;
        if (++ks == p.KW) {
          ks = 0;
          ++kr;
        }
      }
    }
    ++lq;
  };
  auto store_stage = [&](const StageRegs<NW, PL>& R, int buf) {
#pragma unroll
    for (int k = 0; k < NW; ++k) {
      const int t = st0 + k * TSTEP;
      if (t < T) sB[buf][t][spos] = interleave_bytes(R.bw[k]);
    }
#pragma unroll
    for (int pl = 0; pl < PL; ++pl) sA[buf][pl][tid] = R.aw[pl];
    sM[buf][tid] = R.mw;
  };

  float4_t acc[PT][T][4];
#pragma unroll
  for (int pp = 0; pp < PT; ++pp)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int a = 0; a < 4; ++a) acc[pp][t][a] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int wpos = wave * 16 * PT + col;
  auto compute = [&](int buf) {
    half8_t av[PL][4];
    uint32_t ix[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
#pragma unroll
      for (int pl = 0; pl < PL; ++pl) av[pl][a] = __builtin_bit_cast(half8_t, sA[buf][pl][a * 64 + lane]);
      ix[a] = sM[buf][a * 64 + lane];
    }
    uint32_t xb[T][PT];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int pp = 0; pp < PT; ++pp)
        xb[t][pp] = reinterpret_cast<const uint16_t*>(&sB[buf][t][wpos + 16 * pp])[g];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int pp = 0; pp < PT; ++pp) {
        const half16_t bf = expand_bits16(xb[t][pp]);
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int pl = 0; pl < PL; ++pl)
            acc[pp][t][a] = __builtin_amdgcn_smfmac_f32_16x16x64_f16(av[pl][a], bf, acc[pp][t][a], ix[a], 0, 0);
      }
  };

  // Double-buffered LDS: the global loads of chunk q+1 are issued before chunk q is
  // multiplied and written to the other buffer after it.
  StageRegs<NW, PL> R;
  load_next(R);
  store_stage(R, 0);
  __syncthreads();
  for (int q = 0; q < p.nq; ++q) {
    const bool more = q + 1 < p.nq;
    if (more) load_next(R);
    compute(q & 1);
    if (more) store_stage(R, (q & 1) ^ 1);
    __syncthreads();
  }

  const int cob = G * 64 + g * 16;
#pragma unroll
  for (int pp = 0; pp < PT; ++pp) {
    const int m = m0 + wpos + 16 * pp;
    if (m < p.M)
      lif_epilogue<T, OUT_ENC, MODE>(acc[pp], m, p.M, p.F, cob, p.np, p.scale, p.bias, p.enc_scale, p.state, p.out,
                                     p.h_trace, p.x_trace);
  }
}

template <int T, int PT, int PL, int OE, int MODE>
static hipError_t launch_lds_t(const LdsParams& p, hipStream_t s) {
  dim3 grid((unsigned)((p.M + 64 * PT - 1) / (64 * PT)), (unsigned)(p.F / 64));
  hipLaunchKernelGGL((fused_sparse_lds_kernel<T, PT, PL, OE, MODE>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

template <int T, int PT>
static hipError_t launch_lds_pt(const LdsParams& p, int planes, int out_enc, int mode, hipStream_t s) {
  if (out_enc == SENGINE_ENC_BITS && mode == EPI_LIF_HARD) {
    if (planes == 1) return launch_lds_t<T, PT, 1, SENGINE_ENC_BITS, EPI_LIF_HARD>(p, s);
    return launch_lds_t<T, PT, 2, SENGINE_ENC_BITS, EPI_LIF_HARD>(p, s);
  }
  if (out_enc == SENGINE_ENC_BITS && mode == EPI_IF_HARD) {
    if (planes == 1) return launch_lds_t<T, PT, 1, SENGINE_ENC_BITS, EPI_IF_HARD>(p, s);
    return launch_lds_t<T, PT, 2, SENGINE_ENC_BITS, EPI_IF_HARD>(p, s);
  }
  if (planes == 1 && out_enc == SENGINE_ENC_BITS) return launch_lds_t<T, PT, 1, SENGINE_ENC_BITS, EPI_GENERIC>(p, s);
  if (planes == 2 && out_enc == SENGINE_ENC_BITS) return launch_lds_t<T, PT, 2, SENGINE_ENC_BITS, EPI_GENERIC>(p, s);
  if (planes == 1 && out_enc == SENGINE_ENC_F16) return launch_lds_t<T, PT, 1, SENGINE_ENC_F16, EPI_GENERIC>(p, s);
  if (planes == 2 && out_enc == SENGINE_ENC_F16) return launch_lds_t<T, PT, 2, SENGINE_ENC_F16, EPI_GENERIC>(p, s);
  return hipErrorInvalidValue;
}

static int env_int(const char* name, int dflt) {
  const char* e = getenv(name);
  return e ? atoi(e) : dflt;
}

// Positions per workgroup: 64 (PT=1) measured faster than 128 on every config-1 layer
// (more waves in flight, fewer registers); 128 only for T <= 2, where the accumulators are
// small.  SENGINE_AMD_LDS_PT=1|2 overrides (tuning).
static int choose_pt(int T) {
  static const int forced = env_int("SENGINE_AMD_LDS_PT", 0);
  if (forced == 1 || forced == 2) return T > 4 ? 1 : forced;
  return T <= 2 ? 2 : 1;
}

hipError_t launch_fused_bits_lds(const sengine_conv_lif_desc* d, const Geometry& geo, const FusedArgs& a,
                                 hipStream_t stream) {
  LdsParams p;
  p.in = static_cast<const uint8_t*>(a.data);
  p.wvals = static_cast<const u32x4_t*>(a.wvals);
  p.wmeta = static_cast<const uint32_t*>(a.wmeta);
  p.state = a.state;
  p.scale = a.scale;
  p.bias = a.bias;
  p.out = static_cast<uint8_t*>(a.out);
  p.h_trace = a.h_trace;
  p.x_trace = a.x_trace;
  p.B = d->B; p.C = d->C_in; p.H = d->H; p.W = d->W; p.F = d->C_out; p.KW = d->KW;
  p.SH = d->stride_h; p.SW = d->stride_w; p.PH = d->pad_h; p.PW = d->pad_w;
  p.DH = d->dil_h; p.DW = d->dil_w; p.OH = geo.OH; p.OW = geo.OW;
  p.M = (int)geo.M;
  p.nq = (int)(geo.K_red / 64);
  p.in_t_bytes = (int64_t)d->B * d->H * d->W * (d->C_in / 8);
  p.np = make_neuron_params(d->neuron, d->hard_reset, d->tau, d->v_threshold, d->v_reset);
  p.enc_scale = 1.0f / kBitSpikeValue;
  const int pt = choose_pt(d->T);
  const int mode = epilogue_mode(p.np, a.h_trace != nullptr || a.x_trace != nullptr);
  const int pl = d->weight_planes, oe = d->out_enc;
#define SENGINE_LDS_T(TT)                                                                      \
  case TT:                                                                                     \
    return pt == 2 ? launch_lds_pt<TT, 2>(p, pl, oe, mode, stream)                      \
                   : launch_lds_pt<TT, 1>(p, pl, oe, mode, stream);
  switch (d->T) {
    SENGINE_LDS_T(1)
    SENGINE_LDS_T(2)
    SENGINE_LDS_T(4)
    case 8:
      return launch_lds_pt<8, 1>(p, pl, oe, mode, stream);
    default:
      return hipErrorInvalidValue;
  }
#undef SENGINE_LDS_T
}

}  // namespace sengine
