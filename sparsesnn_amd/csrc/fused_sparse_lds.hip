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

#include <stdio.h>

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
  int B, C, H, W, F, KH, KW, SH, SW, PH, PW, DH, DW, OH, OW;
  int M, nq;
  int64_t in_t_bytes;  // bytes of one timestep of input spike bits
  NeuronParams np;
  float enc_scale;
  SewAdd sew;
};

__device__ __forceinline__ uint2 interleave_bytes(uint2 w) {
  // [b0 b1 b2 b3 | b4 b5 b6 b7] -> [b0 b4 b1 b5 | b2 b6 b3 b7]
  return uint2{__builtin_amdgcn_perm(w.y, w.x, 0x05010400u), __builtin_amdgcn_perm(w.y, w.x, 0x07030602u)};
}

// Registers holding one chunk's staged data between its global load and its LDS store.
template <int NW, int GPW, int PL>
struct StageRegs {
  uint2 bw[NW];
  u32x4_t aw[GPW][PL];
  uint32_t mw[GPW];
};

// Workgroup order: hardware dispatches consecutive workgroup ids round-robin over the 8
// XCDs (separate L2s).  Remap so each XCD receives a contiguous run of position tiles,
// keeping the input rows shared by neighbouring tiles in one L2.
__device__ __forceinline__ int xcd_tile(int id, int n) {
  const int per = n >> 3;                 // full tiles per XCD
  if (id >= per * 8) return id;           // ragged tail keeps its id
  return (id & 7) * per + (id >> 3);
}

// T timesteps, PT*64 positions per workgroup, GPW 64-channel output groups per wave,
// PL weight planes, output encoding, epilogue mode, CPS reduction chunks per LDS stage.
template <int T, int PT, int GPW, int PL, int OUT_ENC, int MODE, int CPS>
__global__ __launch_bounds__(256) void fused_sparse_lds_kernel(LdsParams p) {
  constexpr int NPOS = 64 * PT;                  // positions per workgroup
  constexpr int TSTEP = 256 / NPOS;              // timesteps covered by one pass of 256 threads
  constexpr int NW = (T + TSTEP - 1) / TSTEP;    // spike words staged per thread per chunk
  constexpr int NCH = 64 * GPW;                  // output channels per workgroup
  __shared__ uint2 sB[2][CPS][T][NPOS];
  __shared__ u32x4_t sA[2][CPS][GPW][PL][256];
  __shared__ uint32_t sM[2][CPS][GPW][256];
  __shared__ float sCoef[4][NCH];                // folded scale, folded bias, scale, bias

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int col = lane & 15;
  const int G0 = blockIdx.y * GPW;  // first 64-channel output group of this workgroup
  const int m0 = xcd_tile(blockIdx.x, gridDim.x) * NPOS;

  // Folded BN coefficients of this workgroup's channels (written before the first barrier).
  const bool fold = MODE == EPI_LIF_HARD || (MODE == EPI_GENERIC && p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2);
  if (tid < NCH) {
    const float sc = p.scale[G0 * 64 + tid] * p.enc_scale;  // exact: enc_scale is a power of two
    const float bi = p.bias[G0 * 64 + tid];
    sCoef[0][tid] = fold ? sc * p.np.rtau : sc;             // exact: rtau is a power of two
    sCoef[1][tid] = fold ? bi * p.np.rtau : bi;
    sCoef[2][tid] = sc;
    sCoef[3][tid] = bi;
  }

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
  // Taps whose input pixel lies inside the image (bit kr*KW + ks; KH*KW <= 64).
  uint64_t tapmask = 0;
  if (svalid)
    for (int kr = 0; kr < p.KH; ++kr) {
      const int ih = ih0 + kr * p.DH;
      if (ih < 0 || ih >= p.H) continue;
      for (int ks = 0; ks < p.KW; ++ks) {
        const int iw = iw0 + ks * p.DW;
        if (iw >= 0 && iw < p.W) tapmask |= 1ull << (kr * p.KW + ks);
      }
    }
  // Byte offset of tap (0, 0), channel 0, timestep st0 (only dereferenced for valid taps).
  const int64_t off00 = (((int64_t)sb * p.H + ih0) * p.W + iw0) * cbytes + (int64_t)st0 * p.in_t_bytes;
  const int64_t dks = (int64_t)p.DW * cbytes;                       // next tap in a kernel row
  const int64_t dkr = (int64_t)p.DH * p.W * cbytes - p.KW * dks;     // wrap to the next kernel row
  const int64_t tstride = (int64_t)TSTEP * p.in_t_bytes;

  const u32x4_t* wv = p.wvals + (size_t)G0 * p.nq * PL * 256 + tid;
  const uint32_t* wm = p.wmeta + (size_t)G0 * p.nq * 256 + tid;
  const size_t wv_group = (size_t)p.nq * PL * 256, wm_group = (size_t)p.nq * 256;

  // counters of the next chunk to load: q = (tap, c0), uniform in the workgroup
  int lq = 0, tap = 0, ks = 0, c0 = 0;
  int64_t tap_off = 0;
  auto load_chunk = [&](StageRegs<NW, GPW, PL>& R) {
    if (lq < p.nq) {
      const bool ok = (tapmask >> tap) & 1;
      const int64_t base = off00 + tap_off + (c0 >> 3);
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        R.bw[k] = uint2{0u, 0u};
        if (ok && st0 + k * TSTEP < T) R.bw[k] = *reinterpret_cast<const uint2*>(p.in + base + k * tstride);
      }
#pragma unroll
      for (int gg = 0; gg < GPW; ++gg) {
#pragma unroll
        for (int pl = 0; pl < PL; ++pl) R.aw[gg][pl] = wv[gg * wv_group + ((size_t)lq * PL + pl) * 256];
        R.mw[gg] = wm[gg * wm_group + (size_t)lq * 256];
      }
      c0 += 64;
      if (c0 == p.C) {
        c0 = 0;
        ++tap;
        tap_off += dks;
        if (++ks == p.KW) {
          ks = 0;
          tap_off += dkr;
        }
      }
    }
    ++lq;
  };
  auto store_chunk = [&](const StageRegs<NW, GPW, PL>& R, int buf, int c) {
#pragma unroll
    for (int k = 0; k < NW; ++k) {
      const int t = st0 + k * TSTEP;
      if (t < T) sB[buf][c][t][spos] = interleave_bytes(R.bw[k]);
    }
#pragma unroll
    for (int gg = 0; gg < GPW; ++gg) {
#pragma unroll
      for (int pl = 0; pl < PL; ++pl) sA[buf][c][gg][pl][tid] = R.aw[gg][pl];
      sM[buf][c][gg][(tid & 3) * 64 + (tid >> 2)] = R.mw[gg];  // blob [lane][tile] -> LDS [tile][lane]
    }
  };

  float4_t acc[PT][GPW][T][4];
#pragma unroll
  for (int pp = 0; pp < PT; ++pp)
#pragma unroll
    for (int gg = 0; gg < GPW; ++gg)
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int a = 0; a < 4; ++a) acc[pp][gg][t][a] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int wpos = wave * 16 * PT + col;
  auto compute = [&](int buf, int c) {
    half8_t av[GPW][PL][4];
    uint32_t ix[GPW][4];
#pragma unroll
    for (int gg = 0; gg < GPW; ++gg)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
#pragma unroll
        for (int pl = 0; pl < PL; ++pl)
          av[gg][pl][a] = __builtin_bit_cast(half8_t, sA[buf][c][gg][pl][a * 64 + lane]);
        ix[gg][a] = sM[buf][c][gg][a * 64 + lane];
      }
    uint32_t xb[T][PT];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int pp = 0; pp < PT; ++pp)
        xb[t][pp] = reinterpret_cast<const uint16_t*>(&sB[buf][c][t][wpos + 16 * pp])[g];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int pp = 0; pp < PT; ++pp) {
        const half16_t bf = expand_bits16(xb[t][pp]);
#pragma unroll
        for (int gg = 0; gg < GPW; ++gg)
#pragma unroll
          for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int pl = 0; pl < PL; ++pl)
              acc[pp][gg][t][a] =
                  __builtin_amdgcn_smfmac_f32_16x16x64_f16(av[gg][pl][a], bf, acc[pp][gg][t][a], ix[gg][a], 0, 0);
      }
  };

  // Double-buffered LDS stages of CPS chunks: the global loads of stage s+1 are issued
  // before stage s is multiplied and written to the other buffer after it.  (A two-stage
  // deep register prefetch measured slower: the second register set costs occupancy.)
  StageRegs<NW, GPW, PL> R[CPS];
#pragma unroll
  for (int c = 0; c < CPS; ++c) load_chunk(R[c]);
#pragma unroll
  for (int c = 0; c < CPS; ++c) store_chunk(R[c], 0, c);
  __syncthreads();
  const int nstage = (p.nq + CPS - 1) / CPS;
  for (int st = 0; st < nstage; ++st) {
    const int buf = st & 1;
    const bool more = st + 1 < nstage;
    if (more) {
#pragma unroll
      for (int c = 0; c < CPS; ++c) load_chunk(R[c]);
    }
#pragma unroll
    for (int c = 0; c < CPS; ++c)
      if (c == 0 || st * CPS + c < p.nq) compute(buf, c);
    if (more) {
#pragma unroll
      for (int c = 0; c < CPS; ++c) store_chunk(R[c], buf ^ 1, c);
    }
    __syncthreads();
  }

#pragma unroll
  for (int pp = 0; pp < PT; ++pp) {
    const int m = m0 + wpos + 16 * pp;
#pragma unroll
    for (int gg = 0; gg < GPW; ++gg) {
      const int lc = gg * 64 + g * 16;  // workgroup-local channel of this lane's first output
      const EpiCoeffs cf{&sCoef[0][lc], &sCoef[1][lc], &sCoef[2][lc], &sCoef[3][lc]};
      lif_epilogue<T, OUT_ENC, MODE>(acc[pp][gg], m < p.M, m, p.M, p.F, (G0 + gg) * 64 + g * 16, p.np, cf,
                                     p.state, p.out, p.h_trace, p.x_trace, p.sew);
    }
  }
}

static int env_int(const char* name, int dflt) {
  const char* e = getenv(name);
  return e ? atoi(e) : dflt;
}

// Reduction chunks per LDS stage.  2 halves the barriers but the larger staging set pushes
// the kernel to the VGPR limit and measured slower on every layer tried, so 1 is the default;
// SENGINE_AMD_LDS_CPS=2 selects the other variant (tuning; one-plane weights only).
static int choose_cps(int planes) {
  static const int forced = env_int("SENGINE_AMD_LDS_CPS", 0);
  if (planes == 2) return 1;
  return forced == 2 ? 2 : 1;
}

template <int T, int PT, int GPW, int PL, int OE, int MODE>
static hipError_t launch_lds_t(const LdsParams& p, hipStream_t s) {
  dim3 grid((unsigned)((p.M + 64 * PT - 1) / (64 * PT)), (unsigned)(p.F / (64 * GPW)));
  if (PL == 1 && choose_cps(PL) == 2)
    hipLaunchKernelGGL((fused_sparse_lds_kernel<T, PT, GPW, PL, OE, MODE, 2>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((fused_sparse_lds_kernel<T, PT, GPW, PL, OE, MODE, 1>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

template <int T, int PT, int GPW>
static hipError_t launch_lds_pt(const LdsParams& p, int planes, int out_enc, int mode, hipStream_t s) {
  if (out_enc == SENGINE_ENC_BITS && mode == EPI_LIF_HARD) {
    if (planes == 1) return launch_lds_t<T, PT, GPW, 1, SENGINE_ENC_BITS, EPI_LIF_HARD>(p, s);
    return launch_lds_t<T, PT, GPW, 2, SENGINE_ENC_BITS, EPI_LIF_HARD>(p, s);
  }
  if (out_enc == SENGINE_ENC_BITS && mode == EPI_IF_HARD) {
    if (planes == 1) return launch_lds_t<T, PT, GPW, 1, SENGINE_ENC_BITS, EPI_IF_HARD>(p, s);
    return launch_lds_t<T, PT, GPW, 2, SENGINE_ENC_BITS, EPI_IF_HARD>(p, s);
  }
  if (planes == 1 && out_enc == SENGINE_ENC_BITS) return launch_lds_t<T, PT, GPW, 1, SENGINE_ENC_BITS, EPI_GENERIC>(p, s);
  if (planes == 2 && out_enc == SENGINE_ENC_BITS) return launch_lds_t<T, PT, GPW, 2, SENGINE_ENC_BITS, EPI_GENERIC>(p, s);
  if (planes == 1 && out_enc == SENGINE_ENC_F16) return launch_lds_t<T, PT, GPW, 1, SENGINE_ENC_F16, EPI_GENERIC>(p, s);
  if (planes == 2 && out_enc == SENGINE_ENC_F16) return launch_lds_t<T, PT, GPW, 2, SENGINE_ENC_F16, EPI_GENERIC>(p, s);
  return hipErrorInvalidValue;
}


// Positions per workgroup: 64 (PT=1) measured faster than 128 on every config-1 layer
// (more waves in flight, fewer registers); 128 only for T <= 2, where the accumulators are
// small.  SENGINE_AMD_LDS_PT=1|2 overrides (tuning).
static int choose_pt(int T) {
  static const int forced = env_int("SENGINE_AMD_LDS_PT", 0);
  if (forced == 1 || forced == 2) return T > 4 ? 1 : forced;
  return T <= 2 ? 2 : 1;
}

// Output-channel groups (of 64) per wave: 2 halves the spike-bit expansion work per
// SMFMAC (each B fragment feeds 8 instead of 4), at the cost of twice the accumulators and
// half the workgroups.  Used when C_out % 128 == 0 and the grid still holds >= 1 wave per
// SIMD.  SENGINE_AMD_LDS_GPW=1|2 overrides (tuning).
static int choose_gpw(int T, int pt, int64_t M, int F) {
  static const int forced = env_int("SENGINE_AMD_LDS_GPW", 0);
  if (pt != 1 || T > 4 || F % 128 != 0) return 1;
  if (forced == 1 || forced == 2) return forced;
  const int64_t waves = ((M + 63) / 64) * (F / 128) * 4;
  return waves >= 1024 ? 2 : 1;
}

int describe_lds(const sengine_conv_lif_desc* d, const Geometry& geo, int mode, char* buf, size_t len) {
  static const char* const kEpi[] = {"generic", "lif_hard", "if_hard"};
  const int pt = choose_pt(d->T);
  const int gpw = choose_gpw(d->T, pt, geo.M, d->C_out);
  const bool fast = d->out_enc == SENGINE_ENC_BITS && (mode == EPI_LIF_HARD || mode == EPI_IF_HARD);
  return snprintf(buf, len, "lds<T=%d,PT=%d,GPW=%d,planes=%d,out=%s,epi=%s>", d->T, d->T == 8 ? 1 : pt,
                  d->T == 8 ? 1 : gpw, d->weight_planes, d->out_enc == SENGINE_ENC_BITS ? "bits" : "f16",
                  fast ? kEpi[mode] : "generic");
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
  p.B = d->B; p.C = d->C_in; p.H = d->H; p.W = d->W; p.F = d->C_out; p.KH = d->KH; p.KW = d->KW;
  p.SH = d->stride_h; p.SW = d->stride_w; p.PH = d->pad_h; p.PW = d->pad_w;
  p.DH = d->dil_h; p.DW = d->dil_w; p.OH = geo.OH; p.OW = geo.OW;
  p.M = (int)geo.M;
  p.nq = (int)(geo.K_red / 64);
  p.in_t_bytes = (int64_t)d->B * d->H * d->W * (d->C_in / 8);
  p.np = make_neuron_params(d->neuron, d->hard_reset, d->tau, d->v_threshold, d->v_reset);
  p.enc_scale = 1.0f / kBitSpikeValue;
  p.sew = a.sew;
  const int pt = choose_pt(d->T);
  const int gpw = choose_gpw(d->T, pt, geo.M, d->C_out);
  const int mode = epilogue_mode(p.np, a.h_trace != nullptr || a.x_trace != nullptr || a.sew.real_out != nullptr);
  const int pl = d->weight_planes, oe = d->out_enc;
#define SENGINE_LDS_T(TT)                                                                      \
  case TT:                                                                                     \
    if (pt == 2) return launch_lds_pt<TT, 2, 1>(p, pl, oe, mode, stream);                     \
    return gpw == 2 ? launch_lds_pt<TT, 1, 2>(p, pl, oe, mode, stream)                         \
                    : launch_lds_pt<TT, 1, 1>(p, pl, oe, mode, stream);
  switch (d->T) {
    SENGINE_LDS_T(1)
    SENGINE_LDS_T(2)
    SENGINE_LDS_T(4)
    case 8:
      return launch_lds_pt<8, 1, 1>(p, pl, oe, mode, stream);
    default:
      return hipErrorInvalidValue;
  }
#undef SENGINE_LDS_T
}

}  // namespace sengine
