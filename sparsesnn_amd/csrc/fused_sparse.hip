// Fused 2:4-sparse Conv + folded BN + multi-step LIF/IF for gfx950.
//
// Replaces the reference operator conv2d_bn_if_interleaved_kernel
// (sengine/kernels/conv2d_bn_if_t4.py:918-1022) and conv1x1_bn_lif / conv1x1_bn_if
// (sengine/kernels/interleaved_templates.py:28-154).  Same contract: one launch
// processes all T timesteps of a (T*B, H, W, C_in) input; each workgroup owns its
// output tile across every timestep, so the membrane never leaves registers and no
// two workgroups touch the same membrane (unlike the T-batched kernels at
// conv2d_bn_if_t4.py:214-217).
//
// GEMM view: out^T[C_out, M] = W[C_out, K_red] (2:4 sparse along C_in) x act^T[K_red, M]
// with K_red ordered (kh, kw, c_in), c_in fastest — the order of the reference's
// (KH, KW, C_in, F) weight (cuda_graph_runtime.py:233-235) and of its 2:4 groups
// (sparse/utils.py:87-109).  The weights are the sparse A operand of
// v_smfmac_f32_16x16x64_f16; activations are the dense B operand, gathered straight
// from the NHWC input (implicit im2col) and expanded from spike bits in registers.
//
// Work decomposition: workgroup = 4 waves = 64 output channels x 64 output positions
// (positions flattened over (b, oh, ow), as the reference's M_per_t).  Each wave owns
// 64 channels x 16 positions and accumulates all T timesteps at once (T*4 MFMA tiles),
// so every weight fragment fetched is reused T times from registers.  The weight blob
// permutes rows so that lane group g = lane/16 holds output channels 16g..16g+15 of
// its 64-channel group: the epilogue then forms 16 spike bits per lane with no
// cross-lane traffic.
#include "common.h"
#include "epilogue.h"
#include "internal.h"

#include <stdio.h>

namespace sengine {

struct FusedParams {
  const uint8_t* in;
  const half8_t* wvals;
  const uint32_t* wmeta;
  float* state;
  const float* scale;
  const float* bias;
  uint8_t* out;
  float* h_trace;
  float* x_trace;
  int B, C, H, W, F, KW, SH, SW, PH, PW, DH, DW, OH, OW;
  int M;    // B*OH*OW
  int nq;   // K_red / 64
  int64_t in_t_stride;  // pixels per timestep = B*H*W
  int bn_period;        // BN vectors repeat every bn_period output channels (C_out; flat layout: per pixel)
  NeuronParams np;
  float enc_scale;      // 1/value of a spike fed to the MFMA
  SewAdd sew;
};

// Folded BN coefficients of output channels G*64 .. G*64+63 into LDS (see epilogue.h).
__device__ __forceinline__ void load_coeffs(const FusedParams& p, int G, float (&sCoef)[4][64]) {
  const bool fold = p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2;
  if (threadIdx.x < 64) {
    const int c = (G * 64) % p.bn_period + threadIdx.x;
    const float sc = p.scale[c] * p.enc_scale;
    const float bi = p.bias[c];
    sCoef[0][threadIdx.x] = fold ? sc * p.np.rtau : sc;
    sCoef[1][threadIdx.x] = fold ? bi * p.np.rtau : bi;
    sCoef[2][threadIdx.x] = sc;
    sCoef[3][threadIdx.x] = bi;
  }
  __syncthreads();
}

template <int T, int IN_ENC, int OUT_ENC, int PLANES>
__global__ __launch_bounds__(256) void fused_sparse_conv_bn_lif_kernel(FusedParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int col = lane & 15;
  const int G = blockIdx.y;  // 64-channel output group
  const int m = blockIdx.x * 64 + wave * 16 + col;
  // folded BN coefficients of the workgroup's 64 channels (see epilogue.h)
  __shared__ float sCoef[4][64];
  load_coeffs(p, G, sCoef);
  const bool mvalid = m < p.M;
  int b = 0, oh = 0, ow = 0;
  if (mvalid) {
    const int ohw = p.OH * p.OW;
    b = m / ohw;
    const int r = m - b * ohw;
    oh = r / p.OW;
    ow = r - oh * p.OW;
  }

  float4_t acc[T][4];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int a = 0; a < 4; ++a) acc[t][a] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int nq = p.nq;
  const int chunks_per_tap = p.C >> 6;
  const half8_t* wv = p.wvals + (size_t)G * nq * PLANES * 4 * 64 + lane;
  const uint32_t* wm = p.wmeta + (size_t)G * nq * 4 * 64 + lane * 4;  // [q][lane][tile]
  // Byte selector pulling bits [8g, 8g+8) of each 32-bit half of a 64-channel chunk.
  const uint32_t sel = 0x0c0c0000u | ((uint32_t)(4 + g) << 8) | (uint32_t)g;

  for (int q = 0; q < nq; ++q) {
    const int tap = q / chunks_per_tap;
    const int c0 = (q - tap * chunks_per_tap) << 6;
    const int kr = tap / p.KW;
    const int ks = tap - kr * p.KW;
    const int ih = oh * p.SH - p.PH + kr * p.DH;
    const int iw = ow * p.SW - p.PW + ks * p.DW;
    const bool ok = mvalid && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W;
    const int64_t pix0 = ((int64_t)b * p.H + ih) * p.W + iw;

    half8_t av[PLANES][4];
    uint32_t ix[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
#pragma unroll
      for (int pl = 0; pl < PLANES; ++pl) av[pl][a] = wv[((size_t)(q * PLANES + pl) * 4 + a) * 64];
    }
    {
      const u32x4_t m4 = *reinterpret_cast<const u32x4_t*>(wm + (size_t)q * 4 * 64);
#pragma unroll
      for (int a = 0; a < 4; ++a) ix[a] = m4[a];
    }

#pragma unroll
    for (int t = 0; t < T; ++t) {
      half16_t bf;
      const int64_t pix = pix0 + (int64_t)t * p.in_t_stride;
      if (IN_ENC == SENGINE_ENC_BITS) {
        uint2 w = {0u, 0u};
        if (ok) w = *reinterpret_cast<const uint2*>(p.in + pix * (p.C >> 3) + (c0 >> 3));
        bf = expand_bits16(__builtin_amdgcn_perm(w.y, w.x, sel));
      } else {
        half8_t lo = {}, hi = {};
        if (ok) {
          const half8_t* src =
              reinterpret_cast<const half8_t*>(reinterpret_cast<const _Float16*>(p.in) + pix * p.C + c0 + 8 * g);
          lo = src[0];
          hi = src[4];
        }
        bf = concat8(lo, hi);
      }
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int pl = 0; pl < PLANES; ++pl)
          acc[t][a] = __builtin_amdgcn_smfmac_f32_16x16x64_f16(av[pl][a], bf, acc[t][a], ix[a], 0, 0);
    }
  }

  // ---- epilogue: folded BN + T-step neuron, all in registers ----
  if (!mvalid) return;
  const EpiCoeffs cf{&sCoef[0][g * 16], &sCoef[1][g * 16], &sCoef[2][g * 16], &sCoef[3][g * 16]};
  lif_epilogue<T, OUT_ENC, EPI_GENERIC>(acc, true, m, p.M, p.F, G * 64 + g * 16, p.np, cf, p.state, p.out,
                                        p.h_trace, p.x_trace, p.sew);
}

// ---- small-M variant: split-K over the waves of a workgroup --------------------------------
// For layers with few output positions (the flat layout, or small images at small batch),
// 64-position workgroups give a handful of workgroups, each walking the whole reduction
// alone.  Here a workgroup of kSmallWaves waves owns 16 positions x 64 channels x all T;
// wave s accumulates the reduction chunks q = s, s + kSmallWaves, ... (implicit im2col as
// the direct kernel, any geometry), the partial accumulators are summed in LDS in wave
// order (deterministic), and wave 0 runs the epilogue.  Spike-bit input, any T of the
// direct kernel.  Operands are loaded two chunks ahead; the cross-wave sum takes up to
// four timesteps per LDS round.
constexpr int kSmallWaves = 8;
constexpr int64_t kSmallMaxUnits = 128;  // outputs below 128 (64 positions x 64 channels) units

template <int T, int PLANES>
struct SmallOperands {
  half8_t av[PLANES][4];
  uint32_t ix[4];
  uint2 bw[T];
};

// Workgroup (bx, G): positions bx*16 .. bx*16+15, output channels G*64 .. G*64+63.
template <int T, int OUT_ENC, int PLANES, int MODE>
__device__ __forceinline__ void smallm_body(const FusedParams& p, const int bx, const int G) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int col = lane & 15;
  const int m = bx * 16 + col;
  constexpr int TR = T < 4 ? T : 4;  // timesteps per reduction round
  __shared__ float sCoef[4][64];
  __shared__ float4_t red[kSmallWaves][TR][4][64];
  const bool mvalid = m < p.M;
  // Everything the epilogue reads from memory is requested now, next to the first operand
  // loads, instead of after the reduction: BN vectors (to LDS before the first barrier)
  // and, in wave 0, the SEW residual words.
  float csc = 0.f, cbi = 0.f;
  if (threadIdx.x < 64) {
    const int c = (G * 64) % p.bn_period + threadIdx.x;
    csc = p.scale[c];
    cbi = p.bias[c];
  }
  SewRes<T> res;
  if (wave == 0) load_sew_res<T>(p.sew, p.M, m, p.F, G * 64 + g * 16, mvalid, res);

  float4_t acc[T][4];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int a = 0; a < 4; ++a) acc[t][a] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int nq = p.nq;
  // implicit im2col, as the direct kernel: chunk q = (tap, 64 input channels); the lane's
  // spike word is the tap-shifted input pixel of its position (zero outside the image)
  int b = 0, oh = 0, ow = 0;
  if (mvalid) {
    const int ohw = p.OH * p.OW;
    b = m / ohw;
    const int r = m - b * ohw;
    oh = r / p.OW;
    ow = r - oh * p.OW;
  }
  const int cbytes = p.C >> 3;
  const int chunks_per_tap = p.C >> 6;
  const size_t tstride = (size_t)p.in_t_stride * cbytes;
  const half8_t* wv = p.wvals + (size_t)G * nq * PLANES * 4 * 64 + lane;
  const uint32_t* wm = p.wmeta + (size_t)G * nq * 4 * 64 + lane * 4;  // [q][lane][tile]
  const uint32_t sel = 0x0c0c0000u | ((uint32_t)(4 + g) << 8) | (uint32_t)g;

  auto load = [&](int q, SmallOperands<T, PLANES>& o) {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
#pragma unroll
      for (int pl = 0; pl < PLANES; ++pl) o.av[pl][a] = wv[((size_t)(q * PLANES + pl) * 4 + a) * 64];
    }
    {
      const u32x4_t m4 = *reinterpret_cast<const u32x4_t*>(wm + (size_t)q * 4 * 64);
#pragma unroll
      for (int a = 0; a < 4; ++a) o.ix[a] = m4[a];
    }
    const int tap = q / chunks_per_tap;
    const int c0 = q - tap * chunks_per_tap;
    const int kr = tap / p.KW;
    const int ih = oh * p.SH - p.PH + kr * p.DH;
    const int iw = ow * p.SW - p.PW + (tap - kr * p.KW) * p.DW;
    const bool ok = mvalid && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W;
    const uint8_t* src = p.in + (((size_t)b * p.H + (ok ? ih : 0)) * p.W + (ok ? iw : 0)) * cbytes + c0 * 8;
#pragma unroll
    for (int t = 0; t < T; ++t)
      o.bw[t] = ok ? *reinterpret_cast<const uint2*>(src + t * tstride) : uint2{0u, 0u};
  };
  constexpr int S = kSmallWaves;
  constexpr bool DEEP = T * PLANES <= 4;  // two chunks ahead where the registers allow, else one
  SmallOperands<T, PLANES> cur, n1, n2;
  if (wave < nq) load(wave, cur);
  if (DEEP && wave + S < nq) load(wave + S, n1);
  for (int q = wave; q < nq; q += S) {
    if (DEEP) {
      if (q + 2 * S < nq) load(q + 2 * S, n2);
    } else if (q + S < nq) {
      load(q + S, n1);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const half16_t bf = expand_bits16(__builtin_amdgcn_perm(cur.bw[t].y, cur.bw[t].x, sel));
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int pl = 0; pl < PLANES; ++pl)
          acc[t][a] = __builtin_amdgcn_smfmac_f32_16x16x64_f16(cur.av[pl][a], bf, acc[t][a], cur.ix[a], 0, 0);
    }
    cur = n1;
    if (DEEP) n1 = n2;
  }

  if (threadIdx.x < 64) {
    const bool fold = p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2;
    const float sc = csc * p.enc_scale;
    sCoef[0][threadIdx.x] = fold ? sc * p.np.rtau : sc;
    sCoef[1][threadIdx.x] = fold ? cbi * p.np.rtau : cbi;
    sCoef[2][threadIdx.x] = sc;
    sCoef[3][threadIdx.x] = cbi;
  }
  // deterministic cross-wave sum (wave order), TR timesteps per round
#pragma unroll
  for (int t0 = 0; t0 < T; t0 += TR) {
#pragma unroll
    for (int u = 0; u < TR; ++u)
#pragma unroll
      for (int a = 0; a < 4; ++a) red[wave][u][a][lane] = acc[t0 + u][a];
    __syncthreads();
    for (int i = threadIdx.x; i < TR * 4 * 64; i += 64 * S) {
      const int u = i >> 8, a = (i >> 6) & 3, l = i & 63;
      float4_t sum = red[0][u][a][l];
#pragma unroll
      for (int w = 1; w < S; ++w) sum += red[w][u][a][l];
      red[0][u][a][l] = sum;
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int u = 0; u < TR; ++u)
#pragma unroll
        for (int a = 0; a < 4; ++a) acc[t0 + u][a] = red[0][u][a][lane];
    }
    if (t0 + TR < T) __syncthreads();
  }
  if (wave != 0) return;
  const EpiCoeffs cf{&sCoef[0][g * 16], &sCoef[1][g * 16], &sCoef[2][g * 16], &sCoef[3][g * 16]};
  lif_epilogue<T, OUT_ENC, MODE>(acc, mvalid, m, p.M, p.F, G * 64 + g * 16, p.np, cf, p.state, p.out, p.h_trace,
                                 p.x_trace, p.sew, &res);
}

template <int T, int OUT_ENC, int PLANES, int MODE>
__global__ __launch_bounds__(64 * kSmallWaves) void fused_smallm_kernel(FusedParams p) {
  smallm_body<T, OUT_ENC, PLANES, MODE>(p, (int)blockIdx.x, (int)blockIdx.y);
}

// Two convs that read the same input (a residual block's conv1 and its downsample) in one
// grid: channel groups y < g0 are p0's, the rest p1's; position tiles past a conv's M exit.
// Each workgroup runs exactly the code of the single-conv kernel.
template <int T, int OUT_ENC, int PLANES, int MODE>
__global__ __launch_bounds__(64 * kSmallWaves) void fused_smallm_pair_kernel(FusedParams p0, FusedParams p1, int g0) {
  const bool second = (int)blockIdx.y >= g0;
  const FusedParams& p = second ? p1 : p0;
  if ((int)blockIdx.x * 16 >= p.M) return;
  smallm_body<T, OUT_ENC, PLANES, MODE>(p, (int)blockIdx.x, second ? (int)blockIdx.y - g0 : (int)blockIdx.y);
}

template <int T>
static hipError_t launch_smallm(const FusedParams& p, int out_enc, int planes, int mode, hipStream_t s) {
  const dim3 grid((unsigned)((p.M + 15) / 16), (unsigned)(p.F / 64));
  const dim3 block(64 * kSmallWaves);
#define SENGINE_SMALLM_CASE(OE, PL, MD)                  \
  if (out_enc == OE && planes == PL && mode == MD) {     \
    hipLaunchKernelGGL((fused_smallm_kernel<T, OE, PL, MD>), grid, block, 0, s, p); \
    return hipGetLastError();                            \
  }
  SENGINE_SMALLM_CASE(SENGINE_ENC_BITS, 1, EPI_LIF_HARD)
  SENGINE_SMALLM_CASE(SENGINE_ENC_BITS, 1, EPI_IF_HARD)
  SENGINE_SMALLM_CASE(SENGINE_ENC_BITS, 1, EPI_GENERIC)
  SENGINE_SMALLM_CASE(SENGINE_ENC_BITS, 2, EPI_GENERIC)
  SENGINE_SMALLM_CASE(SENGINE_ENC_F16, 1, EPI_GENERIC)
  SENGINE_SMALLM_CASE(SENGINE_ENC_F16, 2, EPI_GENERIC)
#undef SENGINE_SMALLM_CASE
  return hipErrorInvalidValue;
}

template <int T>
static hipError_t launch_smallm_pair(const FusedParams& p0, const FusedParams& p1, int out_enc, int planes, int mode,
                                     hipStream_t s) {
  const int g0 = p0.F / 64;
  const dim3 grid((unsigned)((std::max(p0.M, p1.M) + 15) / 16), (unsigned)(g0 + p1.F / 64));
  const dim3 block(64 * kSmallWaves);
#define SENGINE_SMALLM_PAIR_CASE(OE, PL, MD)                                        \
  if (out_enc == OE && planes == PL && mode == MD) {                               \
    hipLaunchKernelGGL((fused_smallm_pair_kernel<T, OE, PL, MD>), grid, block, 0, s, p0, p1, g0); \
    return hipGetLastError();                                                      \
  }
  SENGINE_SMALLM_PAIR_CASE(SENGINE_ENC_BITS, 1, EPI_LIF_HARD)
  SENGINE_SMALLM_PAIR_CASE(SENGINE_ENC_BITS, 1, EPI_IF_HARD)
  SENGINE_SMALLM_PAIR_CASE(SENGINE_ENC_BITS, 1, EPI_GENERIC)
  SENGINE_SMALLM_PAIR_CASE(SENGINE_ENC_BITS, 2, EPI_GENERIC)
#undef SENGINE_SMALLM_PAIR_CASE
  return hipErrorInvalidValue;
}

template <int T, int IN_ENC, int OUT_ENC, int PLANES>
static hipError_t launch_fused_t(const FusedParams& p, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((fused_sparse_conv_bn_lif_kernel<T, IN_ENC, OUT_ENC, PLANES>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

template <int T>
static hipError_t launch_fused_enc(const FusedParams& p, int in_enc, int out_enc, int planes, dim3 grid,
                                   hipStream_t s) {
#define SENGINE_FUSED_CASE(IE, OE, PL) \
  if (in_enc == IE && out_enc == OE && planes == PL) return launch_fused_t<T, IE, OE, PL>(p, grid, s);
  SENGINE_FUSED_CASE(SENGINE_ENC_BITS, SENGINE_ENC_BITS, 1)
  SENGINE_FUSED_CASE(SENGINE_ENC_BITS, SENGINE_ENC_BITS, 2)
  SENGINE_FUSED_CASE(SENGINE_ENC_BITS, SENGINE_ENC_F16, 1)
  SENGINE_FUSED_CASE(SENGINE_ENC_BITS, SENGINE_ENC_F16, 2)
  SENGINE_FUSED_CASE(SENGINE_ENC_F16, SENGINE_ENC_BITS, 1)
  SENGINE_FUSED_CASE(SENGINE_ENC_F16, SENGINE_ENC_BITS, 2)
  SENGINE_FUSED_CASE(SENGINE_ENC_F16, SENGINE_ENC_F16, 1)
  SENGINE_FUSED_CASE(SENGINE_ENC_F16, SENGINE_ENC_F16, 2)
#undef SENGINE_FUSED_CASE
  return hipErrorInvalidValue;
}

}  // namespace sengine

using namespace sengine;

// Where fused_entry sends a descriptor.
enum FusedRoute { kRouteTiled, kRouteSmall, kRouteDirect };

struct FusedPlan {
  Geometry geo;
  FusedRoute route;
  FusedParams p;  // kRouteSmall / kRouteDirect
  int mode;       // kRouteSmall: epilogue mode
};

// Checks a descriptor and its pointers and picks the kernel.  Small outputs run in the flat
// layout (their weight blob is built that way): the split-K small-M kernel for bit inputs,
// the direct kernel on the flat view otherwise.  Other bit inputs: tile kernel for 3x3 /
// stride 1 / pad 1 and 1x1 / pad 0, the strided halo-tiled kernel for 3x3 / stride 2 / pad 1
// at T = 4, else the LDS-staged kernel (its per-thread tap mask holds up to 64 taps), else the
// direct-gather kernel.
static int plan_fused(const sengine_conv_lif_desc* d, const void* data, const void* blob_values,
                      const void* blob_meta, float* state, const float* bn_scale, const float* bn_bias, void* spikes,
                      float* h_trace, float* x_trace, const SewAdd& sew, FusedPlan& plan) {
  Geometry& geo = plan.geo;
  int rc = check_desc(d, &geo, /*sparse=*/true);
  if (rc) return rc;
  if (!data || !blob_values || !blob_meta || !bn_scale || !bn_bias || !spikes)
    return set_error(-1, "fused_sparse_conv_bn_lif: null data/weight/bn/spikes pointer");
  if (d->T != 1 && d->T != 2 && d->T != 4 && d->T != 8)
    return set_error(-3, "fused_sparse_conv_bn_lif: T must be 1, 2, 4 or 8");
  if (d->in_enc != SENGINE_ENC_BITS && d->in_enc != SENGINE_ENC_F16)
    return set_error(-2, "fused_sparse_conv_bn_lif: in_enc must be BITS or F16");
  if (d->out_enc != SENGINE_ENC_BITS && d->out_enc != SENGINE_ENC_F16)
    return set_error(-2, "fused_sparse_conv_bn_lif: out_enc must be BITS or F16");
  if (geo.M > (1ll << 30)) return set_error(-2, "fused_sparse_conv_bn_lif: B*OH*OW too large");

  const int choice = fused_kernel_choice();
  const bool flat = flat_layout(d, geo);
  // few 64-position x 64-channel work units: split the reduction inside workgroups instead
  const bool small = d->in_enc == SENGINE_ENC_BITS && choice == 0 &&
                     ((geo.M + 63) / 64) * (int64_t)(d->C_out / 64) < kSmallMaxUnits;
  if (!flat && !small && d->in_enc == SENGINE_ENC_BITS && choice != 1 &&
      (((choice == 0 || choice == 3) && tile_eligible(d)) || d->KH * d->KW <= 64)) {
    plan.route = kRouteTiled;
    return 0;
  }
  // fp16 activations (the reference's call() ABI): the tile kernel copies fp16 rows into its
  // LDS layout, as halo tiles (3x3 / s1 / p1), position tiles (1x1 / p0) or, for any other
  // geometry at T = 4, one tap per chunk (the gather form); the rest take the direct-gather kernel
  if (!flat && d->in_enc == SENGINE_ENC_F16 && (choice == 0 || choice == 3) &&
      (tile_eligible(d) || tile_gather_eligible(d))) {
    plan.route = kRouteTiled;
    return 0;
  }

  FusedParams& p = plan.p;
  p.in = static_cast<const uint8_t*>(data);
  p.wvals = static_cast<const half8_t*>(blob_values);
  p.wmeta = static_cast<const uint32_t*>(blob_meta);
  p.state = state;
  p.scale = bn_scale;
  p.bias = bn_bias;
  p.out = static_cast<uint8_t*>(spikes);
  p.h_trace = h_trace;
  p.x_trace = x_trace;
  p.B = d->B; p.C = d->C_in; p.H = d->H; p.W = d->W; p.F = d->C_out; p.KW = d->KW;
  p.SH = d->stride_h; p.SW = d->stride_w; p.PH = d->pad_h; p.PW = d->pad_w;
  p.DH = d->dil_h; p.DW = d->dil_w; p.OH = geo.OH; p.OW = geo.OW;
  p.M = (int)geo.M;
  p.nq = (int)(geo.K_red / 64);
  p.in_t_stride = (int64_t)d->B * d->H * d->W;
  p.np = make_neuron_params(d->neuron, d->hard_reset, d->tau, d->v_threshold, d->v_reset);
  p.enc_scale = d->in_enc == SENGINE_ENC_BITS ? 1.0f / kBitSpikeValue : 1.0f;
  p.sew = sew;
  p.sew.pix_ch = d->C_out;
  p.bn_period = d->C_out;
  if (flat) {  // one position per image: a 1x1 conv over the flattened image
    p.C = d->H * d->W * d->C_in;
    p.F = geo.OH * geo.OW * d->C_out;
    p.H = p.W = p.OH = p.OW = 1;
    p.KW = 1;
    p.SH = p.SW = p.DH = p.DW = 1;
    p.PH = p.PW = 0;
    p.M = d->B;
    p.nq = p.C / 64;
    p.in_t_stride = d->B;
  }
  if ((flat || small) && d->in_enc == SENGINE_ENC_BITS && choice != 1) {
    plan.route = kRouteSmall;
    // fast epilogue modes for the common case (one weight plane, bit output)
    plan.mode = epilogue_mode(p.np, h_trace != nullptr || x_trace != nullptr || sew.real_out != nullptr);
    if (d->weight_planes != 1 || d->out_enc != SENGINE_ENC_BITS) plan.mode = EPI_GENERIC;
  } else {
    plan.route = kRouteDirect;
  }
  return 0;
}

static int fused_entry(const sengine_conv_lif_desc* d, const void* data, const void* blob_values,
                       const void* blob_meta, float* state, const float* bn_scale, const float* bn_bias, void* spikes,
                       float* h_trace, float* x_trace, const SewAdd& sew, hipStream_t stream) {
  FusedPlan plan;
  const int rc = plan_fused(d, data, blob_values, blob_meta, state, bn_scale, bn_bias, spikes, h_trace, x_trace, sew,
                            plan);
  if (rc) return rc;
  if (plan.route == kRouteTiled) {
    const FusedArgs args{data, blob_values, blob_meta, state, bn_scale, bn_bias, spikes, h_trace, x_trace, sew};
    const int choice = fused_kernel_choice();
    if ((choice == 0 || choice == 3) && tile_eligible(d)) return (int)launch_fused_bits_tile(d, plan.geo, args, stream);
    if (d->in_enc == SENGINE_ENC_F16) return (int)launch_fused_f16_gather(d, plan.geo, args, stream);
    if ((choice == 0 || choice == 3) && tile3s_eligible(d))
      return (int)launch_fused_bits_tile3s(d, plan.geo, args, stream);
    return (int)launch_fused_bits_lds(d, plan.geo, args, stream);
  }
  const FusedParams& p = plan.p;
  if (plan.route == kRouteSmall) {
    switch (d->T) {
      case 1: return (int)launch_smallm<1>(p, d->out_enc, d->weight_planes, plan.mode, stream);
      case 2: return (int)launch_smallm<2>(p, d->out_enc, d->weight_planes, plan.mode, stream);
      case 4: return (int)launch_smallm<4>(p, d->out_enc, d->weight_planes, plan.mode, stream);
      default: return (int)launch_smallm<8>(p, d->out_enc, d->weight_planes, plan.mode, stream);
    }
  }
  dim3 grid((unsigned)((p.M + 63) / 64), (unsigned)(p.F / 64));
  hipError_t e;
  switch (d->T) {
    case 1: e = launch_fused_enc<1>(p, d->in_enc, d->out_enc, d->weight_planes, grid, stream); break;
    case 2: e = launch_fused_enc<2>(p, d->in_enc, d->out_enc, d->weight_planes, grid, stream); break;
    case 4: e = launch_fused_enc<4>(p, d->in_enc, d->out_enc, d->weight_planes, grid, stream); break;
    default: e = launch_fused_enc<8>(p, d->in_enc, d->out_enc, d->weight_planes, grid, stream); break;
  }
  return (int)e;
}

// The paired-tail call's checks (shared by the call and its plan): 0, or an error.
static int tail_check(const sengine_conv_lif_desc* d, Geometry& geo, bool traces_or_residual, int& mode,
                      const char* who) {
  int rc = check_desc(d, &geo, true);
  if (rc) return rc;
  if ((rc = check_tail_desc(d, who))) return rc;
  if (traces_or_residual) return set_error(-2, "paired-tail call: no traces, SEW sum or shortcut");
  const NeuronParams np = make_neuron_params(d->neuron, d->hard_reset, d->tau, d->v_threshold, d->v_reset);
  mode = epilogue_mode(np, false);
  if (mode != EPI_LIF_HARD && mode != EPI_IF_HARD)
    return set_error(-2, "paired-tail call: needs a hard-reset IF, or a hard-reset LIF with a power-of-two tau");
  return 0;
}

extern "C" int sengine_amd_fused_plan(const sengine_conv_lif_desc* d, int32_t flags, char* buf, size_t len) {
  if (!d || !buf || len == 0) return set_error(-1, "fused_plan: null descriptor or buffer");
  const bool traces = flags & SENGINE_PLAN_TRACES;
  const bool state = flags & SENGINE_PLAN_STATE;
  const bool shortcut = flags & SENGINE_PLAN_SHORTCUT;
  if (flags & SENGINE_PLAN_TAIL) {
    Geometry geo;
    int mode = 0;
    const bool extra = traces || shortcut || (flags & SENGINE_PLAN_SEW_ADD);
    if (const int rc = tail_check(d, geo, extra, mode, "fused_plan (paired tail)")) return rc;
    const int n = describe_tail(d, geo, mode, state, buf, len);
    if (n < 0 || (size_t)n >= len) return set_error(-2, "fused_plan: buffer too small");
    return 0;
  }
  // never dereferenced: the plan only checks that the pointers are present
  const void* nz = reinterpret_cast<const void*>(static_cast<uintptr_t>(256));
  float* fz = reinterpret_cast<float*>(static_cast<uintptr_t>(256));
  const SewAdd sew{(flags & SENGINE_PLAN_SEW_ADD) ? static_cast<const uint8_t*>(nz) : nullptr, 1, 2, d->C_out,
                   nullptr, shortcut ? fz : nullptr};
  FusedPlan plan;
  const int rc = plan_fused(d, nz, nz, nz, state ? fz : nullptr, fz, fz, fz, traces ? fz : nullptr,
                            traces ? fz : nullptr, sew, plan);
  if (rc) return rc;
  static const char* const kEpi[] = {"generic", "lif_hard", "if_hard"};
  const NeuronParams np = make_neuron_params(d->neuron, d->hard_reset, d->tau, d->v_threshold, d->v_reset);
  const int mode = epilogue_mode(np, traces || shortcut);
  int n;
  if (plan.route == kRouteTiled) {
    const int choice = fused_kernel_choice();
    const bool shortcut_only = shortcut && !traces && !(flags & SENGINE_PLAN_SEW_ADD);
    const FusedArgs fa{nz, nz, nz, state ? fz : nullptr, fz, fz, fz, traces ? fz : nullptr, traces ? fz : nullptr, sew};
    if ((choice == 0 || choice == 3) && tile_eligible(d))
      n = describe_tile(d, plan.geo, mode, shortcut_only, fa, buf, len);
    else if (d->in_enc == SENGINE_ENC_F16)
      n = describe_gather(d, plan.geo, mode, buf, len);
    else if ((choice == 0 || choice == 3) && tile3s_eligible(d))
      n = describe_tile3s(d, plan.geo, mode, buf, len);
    else
      n = describe_lds(d, plan.geo, mode, buf, len);
  } else if (plan.route == kRouteSmall) {
    n = snprintf(buf, len, "smallm<T=%d,planes=%d,out=%s,epi=%s,flat=%d>", d->T, d->weight_planes,
                 d->out_enc == SENGINE_ENC_BITS ? "bits" : "f16", kEpi[plan.mode], flat_layout(d, plan.geo) ? 1 : 0);
  } else {
    n = snprintf(buf, len, "direct<T=%d,in=%s,planes=%d,out=%s,flat=%d>", d->T,
                 d->in_enc == SENGINE_ENC_BITS ? "bits" : "f16", d->weight_planes,
                 d->out_enc == SENGINE_ENC_BITS ? "bits" : "f16", flat_layout(d, plan.geo) ? 1 : 0);
  }
  if (n < 0 || (size_t)n >= len) return set_error(-2, "fused_plan: buffer too small");
  return 0;
}

extern "C" int sengine_amd_fused_sparse_conv_bn_lif(const sengine_conv_lif_desc* d, const void* data,
                                                    const void* blob_values, const void* blob_meta,
                                                    float* state, const float* bn_scale, const float* bn_bias,
                                                    void* spikes, float* h_trace, float* x_trace,
                                                    hipStream_t stream) {
  return fused_entry(d, data, blob_values, blob_meta, state, bn_scale, bn_bias, spikes, h_trace, x_trace,
                     SewAdd{nullptr, 0, 0, 0, nullptr, nullptr}, stream);
}

extern "C" int sengine_amd_fused_sparse_conv_bn_lif_tail(const sengine_conv_lif_desc* d, const void* data,
                                                         const void* blob_values, const void* blob_meta, float* state,
                                                         const float* bn_scale, const float* bn_bias, void* spikes,
                                                         hipStream_t stream) {
  Geometry geo;
  int mode = 0;
  if (const int rc = tail_check(d, geo, false, mode, "fused_sparse_conv_bn_lif_tail")) return rc;
  if (!data || !blob_values || !blob_meta || !bn_scale || !bn_bias || !spikes)
    return set_error(-1, "fused_sparse_conv_bn_lif_tail: null pointer");
  const FusedArgs args{data, blob_values, blob_meta, state, bn_scale, bn_bias, spikes, nullptr, nullptr,
                       SewAdd{nullptr, 0, 0, 0, nullptr, nullptr}};
  return (int)launch_fused_bits_tail(d, geo, args, mode, stream);
}

extern "C" int sengine_amd_fused_sparse_conv_bn_lif_split(const sengine_conv_lif_desc* d, const void* data,
                                                          const void* blob_values, const void* blob_meta,
                                                          float* state, const float* bn_scale, const float* bn_bias,
                                                          void* spikes, int32_t split_channels, hipStream_t stream) {
  if (!d) return set_error(-1, "fused_split: null descriptor");
  if (d->out_enc != SENGINE_ENC_BITS) return set_error(-2, "fused_split: spike-bit output only");
  if (split_channels < 64 || split_channels % 64 != 0)
    return set_error(-2, "fused_split: split_channels must be a positive multiple of 64");
  Geometry geo;
  if (const int rc = check_desc(d, &geo, true)) return rc;
  if (flat_layout(d, geo)) return set_error(-2, "fused_split: not available for the flat small-output layout");
  SewAdd sew{nullptr, 0, 0, 0, nullptr, nullptr};
  sew.split_c = split_channels;
  sew.split_bytes = (int64_t)d->T * geo.M * split_channels / 8;
  return fused_entry(d, data, blob_values, blob_meta, state, bn_scale, bn_bias, spikes, nullptr, nullptr, sew, stream);
}

extern "C" int sengine_amd_fused_sparse_conv_bn_lif_pair(const sengine_conv_lif_desc* d0,
                                                         const sengine_conv_lif_desc* d1, const void* data,
                                                         const void* values0, const void* meta0,
                                                         const float* bn_scale0, const float* bn_bias0, void* spikes0,
                                                         const void* values1, const void* meta1,
                                                         const float* bn_scale1, const float* bn_bias1, void* spikes1,
                                                         hipStream_t stream) {
  if (!d0 || !d1) return set_error(-1, "fused_sparse_conv_bn_lif_pair: null descriptor");
  if (d0->T != d1->T || d0->B != d1->B || d0->C_in != d1->C_in || d0->H != d1->H || d0->W != d1->W ||
      d0->in_enc != d1->in_enc)
    return set_error(-2, "fused_sparse_conv_bn_lif_pair: the two convs must read the same input (T, B, C_in, H, W, "
                         "in_enc)");
  const SewAdd none{nullptr, 0, 0, 0, nullptr, nullptr};
  FusedPlan a, b;
  int rc = plan_fused(d0, data, values0, meta0, nullptr, bn_scale0, bn_bias0, spikes0, nullptr, nullptr, none, a);
  if (rc) return rc;
  rc = plan_fused(d1, data, values1, meta1, nullptr, bn_scale1, bn_bias1, spikes1, nullptr, nullptr, none, b);
  if (rc) return rc;
  if (a.route == kRouteSmall && b.route == kRouteSmall && a.mode == b.mode && d0->out_enc == d1->out_enc &&
      d0->weight_planes == d1->weight_planes) {
    switch (d0->T) {
      case 1: return (int)launch_smallm_pair<1>(a.p, b.p, d0->out_enc, d0->weight_planes, a.mode, stream);
      case 2: return (int)launch_smallm_pair<2>(a.p, b.p, d0->out_enc, d0->weight_planes, a.mode, stream);
      case 4: return (int)launch_smallm_pair<4>(a.p, b.p, d0->out_enc, d0->weight_planes, a.mode, stream);
      default: return (int)launch_smallm_pair<8>(a.p, b.p, d0->out_enc, d0->weight_planes, a.mode, stream);
    }
  }
  rc = fused_entry(d0, data, values0, meta0, nullptr, bn_scale0, bn_bias0, spikes0, nullptr, nullptr, none, stream);
  if (rc) return rc;
  return fused_entry(d1, data, values1, meta1, nullptr, bn_scale1, bn_bias1, spikes1, nullptr, nullptr, none, stream);
}

extern "C" int sengine_amd_fused_sparse_conv_bn_lif_add(const sengine_conv_lif_desc* d, const void* data,
                                                        const void* blob_values, const void* blob_meta,
                                                        float* state, const float* bn_scale, const float* bn_bias,
                                                        const void* residual, int32_t residual_planes, void* out,
                                                        int32_t out_planes, hipStream_t stream) {
  if (!d) return set_error(-1, "fused_sparse_conv_bn_lif_add: null descriptor");
  if (!residual) return set_error(-1, "fused_sparse_conv_bn_lif_add: null residual");
  if (d->out_enc == SENGINE_ENC_F16) {  // fp16 output: out = spike + residual as fp16
    if (d->C_out % 32 != 0) return set_error(-2, "fused_sparse_conv_bn_lif_add: C_out % 32 != 0");
    if (residual_planes == 0)  // fp16 residual stream
      return fused_entry(d, data, blob_values, blob_meta, state, bn_scale, bn_bias, out, nullptr, nullptr,
                         SewAdd{nullptr, 0, 0, d->C_out, nullptr, nullptr, static_cast<const _Float16*>(residual)},
                         stream);
    if (residual_planes < 1 || residual_planes > kMaxPlanes)
      return set_error(-2, "fused_sparse_conv_bn_lif_add: need 0 <= residual_planes <= 5 with fp16 output");
    return fused_entry(d, data, blob_values, blob_meta, state, bn_scale, bn_bias, out, nullptr, nullptr,
                       SewAdd{static_cast<const uint8_t*>(residual), residual_planes, residual_planes, d->C_out,
                              nullptr, nullptr, nullptr},
                       stream);
  }
  if (d->out_enc != SENGINE_ENC_BITS) return set_error(-2, "fused_sparse_conv_bn_lif_add: out_enc must be BITS or F16");
  if (residual_planes < 1 || residual_planes > kMaxPlanes || out_planes < residual_planes || out_planes > kMaxPlanes)
    return set_error(-2, "fused_sparse_conv_bn_lif_add: need 1 <= residual_planes <= out_planes <= 5");
  if (d->C_out % 32 != 0) return set_error(-2, "fused_sparse_conv_bn_lif_add: C_out % 32 != 0");
  return fused_entry(d, data, blob_values, blob_meta, state, bn_scale, bn_bias, out, nullptr, nullptr,
                     SewAdd{static_cast<const uint8_t*>(residual), residual_planes, out_planes, d->C_out, nullptr,
                            nullptr},
                     stream);
}

extern "C" int sengine_amd_fused_sparse_conv_bn_add_neuron(const sengine_conv_lif_desc* d, const void* data,
                                                           const void* blob_values, const void* blob_meta,
                                                           float* state, const float* bn_scale, const float* bn_bias,
                                                           const float* residual, float* real_out, void* spikes,
                                                           hipStream_t stream) {
  if (!d) return set_error(-1, "fused_sparse_conv_bn_add_neuron: null descriptor");
  if (!real_out) return set_error(-1, "fused_sparse_conv_bn_add_neuron: null real_out");
  return fused_entry(d, data, blob_values, blob_meta, state, bn_scale, bn_bias, spikes, nullptr, nullptr,
                     SewAdd{nullptr, 0, 0, 0, residual, real_out}, stream);
}
