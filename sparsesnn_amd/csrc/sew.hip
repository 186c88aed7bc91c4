// The layers of a SEW-ResNet around the fused Conv+BN+LIF op (models/sewresnet.py:123-210):
// the dense stem convolution on image pixels, the neuron over the stem output repeated over
// T, max-pooling of spike bits, and the pooled / time-averaged Linear head.  All of them
// are small next to the fused convolutions; they are HBM- or launch-bound.
#include "common.h"
#include "internal.h"

namespace sengine {

// ---- stem: dense fp32 convolution (any kernel / stride / pad) + folded BN ----------------
// x: NCHW fp32 images (N, C_in, H, W) (the reference feeds the raw 4-D batch to conv1,
// models/sewresnet.py:199); w: OIHW or HWIO fp32; out: NHWC fp32 (N, OH, OW, C_out);
// accumulation in (c_in, kh, kw) order in fp32 like the reference's CPU conv.
// Fast path (HWIO, kernel <= 64 taps, C_in*KH*KW*C_out <= 16K floats): the workgroup stages
// all weights in LDS once; each thread computes 16 output channels of one pixel, so every
// input value it loads feeds 16 FMAs and the weight reads are LDS broadcasts.  Generic
// path: one output value per thread.
struct StemParams {
  const float* x;
  const float* w;
  const float* scale;
  const float* bias;
  float* out;
  int N, C, H, W, F, KH, KW, SH, SW, PH, PW, OH, OW;
  // fused neuron + max-pool (stem_conv_bn_lds_kernel<KW, true>)
  uint16_t* spikes;  // (T, N, OH, OW) x F bits, or null
  uint16_t* pooled;  // (T, N, POH, POW) x F bits
  int T, PK, PS, PP, POH, POW;
  NeuronParams np;
};

constexpr int kStemPix = 256;        // output pixels (of one image) per workgroup, one per thread
constexpr int kStemLdsInput = 12288; // staged, zero-padded input floats
constexpr int kStemLdsW = 4096;      // staged weights of the workgroup's 16 channels

// Workgroup = (image n, block of kStemPix output pixels in (oh, ow) order, 16-channel group
// fg); thread = one output pixel x 16 channels.  The workgroup stages the input rows the
// block reads, with the padding as zeros, and its 16 channels' HWIO weights in LDS; the tap
// loop then has no bounds checks, the weight reads are LDS broadcasts, and with KW_ known
// at compile time a whole tap row's reads are issued before its FMAs.
constexpr int kStemMaxT = 16;  // fused variant: spike words of all T kept in LDS for the pool

template <int KW_, bool FUSE>
__global__ __launch_bounds__(256) void stem_conv_bn_lds_kernel(StemParams p) {
  __shared__ float sx[kStemLdsInput];
  __shared__ float4 sw4[kStemLdsW / 4];
  __shared__ uint16_t sspk[FUSE ? kStemMaxT * kStemPix : 1];
  const int KW = KW_ > 0 ? KW_ : p.KW;
  const int fgroups = p.F / 16;
  const int pblocks = (p.OH * p.OW + kStemPix - 1) / kStemPix;
  const int fg = blockIdx.x % fgroups;
  const int pb = (blockIdx.x / fgroups) % pblocks;
  const int n = blockIdx.x / (fgroups * pblocks);
  const int pix0 = pb * kStemPix;
  const int oh_first = pix0 / p.OW;
  const int oh_last = min(p.OH - 1, (pix0 + kStemPix - 1) / p.OW);
  const int ih0 = oh_first * p.SH - p.PH;
  const int nrows = (oh_last - oh_first) * p.SH + p.KH;
  const int WP = p.W + 2 * p.PW;  // padded row
  // weights: tap-major (kh, kw, c), 16 channels of group fg each, as 4 float4
  const int ntap = p.KH * KW * p.C;
  for (int i = threadIdx.x; i < ntap * 4; i += blockDim.x)
    sw4[i] = *reinterpret_cast<const float4*>(p.w + (int64_t)(i >> 2) * p.F + fg * 16 + (i & 3) * 4);
  const int nx = p.C * nrows * WP;
  for (int i0 = threadIdx.x; i0 < nx; i0 += 8 * blockDim.x) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * blockDim.x;
      const int c = i / (nrows * WP);
      const int rem = i - c * (nrows * WP);
      const int rr = rem / WP;
      const int ih = ih0 + rr;
      const int iw = rem - rr * WP - p.PW;
      v[u] = (i < nx && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W)
                 ? p.x[(((int64_t)n * p.C + c) * p.H + ih) * p.W + iw]
                 : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (i0 + u * blockDim.x < nx) sx[i0 + u * blockDim.x] = v[u];
  }
  __syncthreads();
  const int pix_ = pix0 + threadIdx.x;
  const bool valid = pix_ < p.OH * p.OW;
  if (!FUSE && !valid) return;
  const int pix = valid ? pix_ : pix0;  // the fused variant keeps every thread for its barrier
  const int oh = pix / p.OW;
  const int ow = pix - oh * p.OW;
  const float* xb = &sx[(oh - oh_first) * p.SH * WP + ow * p.SW];
  float acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.f;
  for (int c = 0; c < p.C; ++c)
    for (int kh = 0; kh < p.KH; ++kh) {
      const float* xr = xb + (c * nrows + kh) * WP;
      const float4* wr = sw4 + ((kh * KW) * p.C + c) * 4;
      float xv[KW_ > 0 ? KW_ : 1];
      float4 wv[KW_ > 0 ? KW_ : 1][4];
      if (KW_ > 0) {
#pragma unroll
        for (int kw = 0; kw < (KW_ > 0 ? KW_ : 1); ++kw) {
          xv[kw] = xr[kw];
#pragma unroll
          for (int q = 0; q < 4; ++q) wv[kw][q] = wr[kw * p.C * 4 + q];
        }
#pragma unroll
        for (int kw = 0; kw < (KW_ > 0 ? KW_ : 1); ++kw)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            acc[4 * q + 0] = __builtin_fmaf(xv[kw], wv[kw][q].x, acc[4 * q + 0]);
            acc[4 * q + 1] = __builtin_fmaf(xv[kw], wv[kw][q].y, acc[4 * q + 1]);
            acc[4 * q + 2] = __builtin_fmaf(xv[kw], wv[kw][q].z, acc[4 * q + 2]);
            acc[4 * q + 3] = __builtin_fmaf(xv[kw], wv[kw][q].w, acc[4 * q + 3]);
          }
      } else {
        for (int kw = 0; kw < KW; ++kw) {
          const float x1 = xr[kw];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float4 w1 = wr[kw * p.C * 4 + q];
            acc[4 * q + 0] = __builtin_fmaf(x1, w1.x, acc[4 * q + 0]);
            acc[4 * q + 1] = __builtin_fmaf(x1, w1.y, acc[4 * q + 1]);
            acc[4 * q + 2] = __builtin_fmaf(x1, w1.z, acc[4 * q + 2]);
            acc[4 * q + 3] = __builtin_fmaf(x1, w1.w, acc[4 * q + 3]);
          }
        }
      }
    }
  const float* sc = p.scale + fg * 16;
  const float* bi = p.bias + fg * 16;
  if (!FUSE) {
    float* o = p.out + (((int64_t)n * p.OH + oh) * p.OW + ow) * p.F + fg * 16;
#pragma unroll
    for (int j = 0; j < 16; j += 4)
      *reinterpret_cast<float4*>(o + j) =
          float4{__builtin_fmaf(acc[j], sc[j], bi[j]), __builtin_fmaf(acc[j + 1], sc[j + 1], bi[j + 1]),
                 __builtin_fmaf(acc[j + 2], sc[j + 2], bi[j + 2]), __builtin_fmaf(acc[j + 3], sc[j + 3], bi[j + 3])};
    return;
  }
  // The neuron on the stem output repeated over T (models/sewresnet.py:201-202), the same
  // arithmetic as repeat_neuron_kernel: 16 spike bits per t for this pixel.
  float xf[16], v[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float x = __builtin_fmaf(acc[j], sc[j], bi[j]);
    xf[j] = (p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2) ? x * p.np.rtau : x;  // exact
    v[j] = 0.f;
  }
  const int npix = p.OH * p.OW;
  const int fw = p.F / 16;  // 16-bit spike words per pixel
  for (int t = 0; t < p.T; ++t) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float h = neuron_charge(p.np, v[j], xf[j]);
      const bool spike = h >= p.np.vth;
      v[j] = neuron_reset(p.np, h, spike);
      word |= (uint32_t)spike << j;
    }
    sspk[t * kStemPix + threadIdx.x] = (uint16_t)word;
    if (p.spikes && valid) p.spikes[((int64_t)(t * p.N + n) * npix + pix) * fw + fg] = (uint16_t)word;
  }
  __syncthreads();
  // max-pool of the spikes (models/sewresnet.py:143,203): OR over the in-image taps
  const int npool = p.POH * p.POW;
  for (int i = threadIdx.x; i < p.T * npool; i += blockDim.x) {
    const int t = i / npool;
    const int q = i - t * npool;
    const int ph = q / p.POW;
    const int pw = q - ph * p.POW;
    uint32_t m = 0;
    for (int kh = 0; kh < p.PK; ++kh) {
      const int ih = ph * p.PS - p.PP + kh;
      if (ih < 0 || ih >= p.OH) continue;
      for (int kw = 0; kw < p.PK; ++kw) {
        const int iw = pw * p.PS - p.PP + kw;
        if (iw >= 0 && iw < p.OW) m |= sspk[t * kStemPix + ih * p.OW + iw];
      }
    }
    p.pooled[((int64_t)(t * p.N + n) * npool + q) * fw + fg] = (uint16_t)m;
  }
}

template <int HWIO>
__global__ __launch_bounds__(256) void stem_conv_bn_kernel(StemParams p) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.N * p.OH * p.OW * p.F;
  if (i >= total) return;
  const int f = (int)(i % p.F);
  int64_t r = i / p.F;
  const int ow = (int)(r % p.OW);
  r /= p.OW;
  const int oh = (int)(r % p.OH);
  const int n = (int)(r / p.OH);
  float acc = 0.f;
  for (int c = 0; c < p.C; ++c) {
    const float* xc = p.x + ((int64_t)n * p.C + c) * p.H * p.W;
    for (int kh = 0; kh < p.KH; ++kh) {
      const int ih = oh * p.SH - p.PH + kh;
      if (ih < 0 || ih >= p.H) continue;
      for (int kw = 0; kw < p.KW; ++kw) {
        const int iw = ow * p.SW - p.PW + kw;
        if (iw < 0 || iw >= p.W) continue;
        const float wv = HWIO ? p.w[(((int64_t)kh * p.KW + kw) * p.C + c) * p.F + f]
                              : p.w[(((int64_t)f * p.C + c) * p.KH + kh) * p.KW + kw];
        acc = __builtin_fmaf(xc[ih * p.W + iw], wv, acc);
      }
    }
  }
  p.out[i] = __builtin_fmaf(acc, p.scale[f], p.bias[f]);
}

// ---- neuron over an input repeated at every timestep (models/sewresnet.py:201-202) -------
struct RepeatNeuronParams {
  const float* x;  // n values, the same at every t
  uint32_t* out;   // spike bits (T, n)
  int64_t n;
  int T;
  NeuronParams np;
};

__global__ __launch_bounds__(256) void repeat_neuron_kernel(RepeatNeuronParams p) {
  const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool valid = s < p.n;
  const int lane = threadIdx.x & 63;
  const float x = valid ? p.x[s] : 0.f;
  float xf = x;
  if (p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2) xf = x * p.np.rtau;  // exact
  float v = 0.f;
  for (int t = 0; t < p.T; ++t) {
    const float h = neuron_charge(p.np, v, xf);
    const bool spike = valid && h >= p.np.vth;
    v = neuron_reset(p.np, h, spike);
    const uint64_t mask = __ballot(spike);
    // n % 32 == 0: a 32-lane half-wave is one output word when its first lane is valid
    if ((lane & 31) == 0 && valid) p.out[((int64_t)t * p.n + s) >> 5] = (uint32_t)(mask >> (lane & 32));
  }
}

// ---- max-pooling of spike bits: the max of {0,1} values is their OR ----------------------
// (SeqToANNContainer(MaxPool2d(k, s, p)), models/sewresnet.py:143,203; padding never wins a
// max, so out-of-image taps are skipped).  One thread per (image-timestep, oh, ow, 32-bit word).
struct PoolParams {
  const uint32_t* in;
  uint32_t* out;
  int NT, H, W, CW, K, S, P, OH, OW;  // CW: 32-bit words per pixel
};

__global__ __launch_bounds__(256) void maxpool_bits_kernel(PoolParams p) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.NT * p.OH * p.OW * p.CW;
  if (i >= total) return;
  const int cw = (int)(i % p.CW);
  int64_t r = i / p.CW;
  const int ow = (int)(r % p.OW);
  r /= p.OW;
  const int oh = (int)(r % p.OH);
  const int64_t nt = r / p.OH;
  uint32_t acc = 0;
  for (int kh = 0; kh < p.K; ++kh) {
    const int ih = oh * p.S - p.P + kh;
    if (ih < 0 || ih >= p.H) continue;
    for (int kw = 0; kw < p.K; ++kw) {
      const int iw = ow * p.S - p.P + kw;
      if (iw < 0 || iw >= p.W) continue;
      acc |= p.in[((nt * p.H + ih) * p.W + iw) * p.CW + cw];
    }
  }
  p.out[i] = acc;
}

// ---- head: global average pool per timestep, mean over T, Linear ------------------------
// (models/sewresnet.py:208-210; models/msresnet.py:155-160).  in: integer activations as
// `planes` bit planes, NHWC with planes*C channels, (T*B, HW) positions.  Workgroup (image,
// slice of the outputs): the per-channel sums are exact integers, counted once per
// workgroup -- thread (word column wi, position slice) walks its slice of the T*HW positions
// with coalesced word reads and keeps 32 bit counters in registers, then adds them into LDS
// -- and scaled once into fp32 features; each wave then owns HEAD_OPW outputs at a time
// (looping over the workgroup's slice of the outputs), its lanes split the reduction over C
// (coalesced reads of the Linear weight rows) and a cross-lane sum finishes each output.
constexpr int HEAD_OPW = 4;        // outputs per wave and pass
constexpr int HEAD_MAX_PC = 8192;  // planes * C held as integer counters in LDS
struct HeadParams {
  const uint32_t* in;
  const float* w;  // (N_out, C) fp32, nn.Linear layout
  const float* b;  // (N_out)
  float* out;      // (B, N_out)
  int T, B, HW, C, planes, N_out;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__global__ __launch_bounds__(256) void sew_head_kernel(HeadParams p) {
  __shared__ int cnt[HEAD_MAX_PC];
  __shared__ float feat[HEAD_MAX_PC];
  const int bimg = blockIdx.x;
  const int words = p.planes * p.C / 32;
  const int npos = p.T * p.HW;  // (t, s) positions of this image
  for (int i = threadIdx.x; i < p.planes * p.C; i += blockDim.x) cnt[i] = 0;
  __syncthreads();
  const int per = words < (int)blockDim.x ? words : (int)blockDim.x;  // word columns per pass
  const int nslice = (int)blockDim.x / per;
  const int slice = (int)threadIdx.x / per;
  for (int wbase = 0; wbase < words; wbase += per) {
    const int wi = wbase + (int)threadIdx.x % per;
    if (slice >= nslice || wi >= words) continue;
    uint32_t c32[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) c32[j] = 0;
    for (int q = slice; q < npos; q += nslice) {
      const int t = q / p.HW;
      const uint32_t w = p.in[((int64_t)(t * p.B + bimg) * p.HW + (q - t * p.HW)) * words + wi];
#pragma unroll
      for (int j = 0; j < 32; ++j) c32[j] += (w >> j) & 1u;
    }
#pragma unroll
    for (int j = 0; j < 32; ++j)
      if (c32[j]) atomicAdd(&cnt[wi * 32 + j], (int)c32[j]);
  }
  __syncthreads();
  // channel c of plane pl is bit (pl*C + c) of a position's words
  for (int c = threadIdx.x; c < p.C; c += blockDim.x) {
    int sum = 0;
    for (int pl = 0; pl < p.planes; ++pl) sum += cnt[pl * p.C + c] << pl;
    // mean over HW then over T: both exact or one rounding for the integer sums here
    feat[c] = ((float)sum / (float)p.HW) / (float)p.T;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int nwave_out = (int)(blockDim.x >> 6) * HEAD_OPW;  // outputs per pass of the workgroup
  for (int base = blockIdx.y * nwave_out; base < p.N_out; base += gridDim.y * nwave_out) {
    const int o0 = base + (int)(threadIdx.x >> 6) * HEAD_OPW;
    float acc[HEAD_OPW];
    const float* wrow[HEAD_OPW];
#pragma unroll
    for (int j = 0; j < HEAD_OPW; ++j) {
      acc[j] = 0.f;
      wrow[j] = p.w + (int64_t)min(o0 + j, p.N_out - 1) * p.C;  // rows past N_out: computed, not stored
    }
    // branch-free body, so the unrolled iterations' loads are all in flight together
#pragma unroll 8
    for (int c = lane; c < p.C; c += 64) {
      const float f = feat[c];
#pragma unroll
      for (int j = 0; j < HEAD_OPW; ++j) acc[j] = __builtin_fmaf(f, wrow[j][c], acc[j]);
    }
#pragma unroll
    for (int j = 0; j < HEAD_OPW; ++j) {
      const float v = wave_sum(acc[j]);
      if (lane == 0 && o0 + j < p.N_out) p.out[(int64_t)bimg * p.N_out + o0 + j] = v + p.b[o0 + j];
    }
  }
}

}  // namespace sengine

using namespace sengine;

extern "C" int sengine_amd_stem_conv_bn(const sengine_conv_lif_desc* d, const float* x, const float* weight,
                                        int32_t w_layout, const float* bn_scale, const float* bn_bias, float* out,
                                        hipStream_t stream) {
  if (!d || !x || !weight || !bn_scale || !bn_bias || !out) return set_error(-1, "stem_conv_bn: null pointer");
  if (w_layout != SENGINE_WLAYOUT_OIHW && w_layout != SENGINE_WLAYOUT_HWIO)
    return set_error(-2, "stem_conv_bn: w_layout must be OIHW or HWIO");
  if (d->B < 1 || d->C_in < 1 || d->H < 1 || d->W < 1 || d->C_out < 1 || d->KH < 1 || d->KW < 1 || d->stride_h < 1 ||
      d->stride_w < 1 || d->pad_h < 0 || d->pad_w < 0)
    return set_error(-2, "stem_conv_bn: invalid shape fields");
  if (d->dil_h != 1 || d->dil_w != 1) return set_error(-2, "stem_conv_bn: dilation must be 1");
  StemParams p;
  p.x = x; p.w = weight; p.scale = bn_scale; p.bias = bn_bias; p.out = out;
  p.N = d->B; p.C = d->C_in; p.H = d->H; p.W = d->W; p.F = d->C_out; p.KH = d->KH; p.KW = d->KW;
  p.SH = d->stride_h; p.SW = d->stride_w; p.PH = d->pad_h; p.PW = d->pad_w;
  p.OH = (d->H + 2 * d->pad_h - d->KH) / d->stride_h + 1;
  p.OW = (d->W + 2 * d->pad_w - d->KW) / d->stride_w + 1;
  if (p.OH < 1 || p.OW < 1) return set_error(-2, "stem_conv_bn: empty output");
  const int64_t total = (int64_t)p.N * p.OH * p.OW * p.F;
  // staged rows of one block of kStemPix output pixels: at most ceil(kStemPix / OW) + 1 output rows
  const int64_t max_orows = std::min<int64_t>(p.OH, (kStemPix + p.OW - 1) / p.OW + 1);
  const int64_t staged = (int64_t)p.C * ((max_orows - 1) * p.SH + p.KH) * (p.W + 2 * p.PW);
  if (w_layout == SENGINE_WLAYOUT_HWIO && p.F % 16 == 0 && staged <= kStemLdsInput &&
      (int64_t)p.KH * p.KW * p.C * 16 <= kStemLdsW) {
    const int64_t blocks = (int64_t)p.N * ((p.OH * p.OW + kStemPix - 1) / kStemPix) * (p.F / 16);
    if (p.KW == 7)
      hipLaunchKernelGGL((stem_conv_bn_lds_kernel<7, false>), dim3((unsigned)blocks), dim3(kStemPix), 0, stream, p);
    else
      hipLaunchKernelGGL((stem_conv_bn_lds_kernel<0, false>), dim3((unsigned)blocks), dim3(kStemPix), 0, stream, p);
  } else if (w_layout == SENGINE_WLAYOUT_HWIO)
    hipLaunchKernelGGL(stem_conv_bn_kernel<1>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(stem_conv_bn_kernel<0>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_stem_conv_bn_lif_pool(const sengine_conv_lif_desc* d, const float* x, const float* weight,
                                                 const float* bn_scale, const float* bn_bias, int32_t pool_k,
                                                 int32_t pool_stride, int32_t pool_pad, uint32_t* spikes,
                                                 uint32_t* pooled, hipStream_t stream) {
  if (!d || !x || !weight || !bn_scale || !bn_bias || !pooled)
    return set_error(-1, "stem_conv_bn_lif_pool: null pointer");
  if (d->B < 1 || d->C_in < 1 || d->H < 1 || d->W < 1 || d->C_out < 16 || d->C_out % 32 != 0 || d->KH < 1 ||
      d->KW < 1 || d->stride_h < 1 || d->stride_w < 1 || d->pad_h < 0 || d->pad_w < 0 || d->dil_h != 1 ||
      d->dil_w != 1)
    return set_error(-2, "stem_conv_bn_lif_pool: invalid shape fields (C_out % 32 == 0, dilation 1)");
  if (d->T < 1 || d->T > kStemMaxT) return set_error(-2, "stem_conv_bn_lif_pool: 1 <= T <= 16");
  if (const char* why = neuron_invalid(d->neuron, d->tau)) return set_error(-2, why);
  if (pool_k < 1 || pool_stride < 1 || pool_pad < 0 || 2 * pool_pad > pool_k)
    return set_error(-2, "stem_conv_bn_lif_pool: pool needs k >= 1, stride >= 1, 0 <= pad <= k/2");
  StemParams p{};
  p.x = x; p.w = weight; p.scale = bn_scale; p.bias = bn_bias; p.out = nullptr;
  p.N = d->B; p.C = d->C_in; p.H = d->H; p.W = d->W; p.F = d->C_out; p.KH = d->KH; p.KW = d->KW;
  p.SH = d->stride_h; p.SW = d->stride_w; p.PH = d->pad_h; p.PW = d->pad_w;
  p.OH = (d->H + 2 * d->pad_h - d->KH) / d->stride_h + 1;
  p.OW = (d->W + 2 * d->pad_w - d->KW) / d->stride_w + 1;
  if (p.OH < 1 || p.OW < 1) return set_error(-2, "stem_conv_bn_lif_pool: empty output");
  p.POH = (p.OH + 2 * pool_pad - pool_k) / pool_stride + 1;
  p.POW = (p.OW + 2 * pool_pad - pool_k) / pool_stride + 1;
  if (p.POH < 1 || p.POW < 1) return set_error(-2, "stem_conv_bn_lif_pool: empty pooled output");
  // one workgroup holds a whole image's stem output for its 16 channels
  const int64_t staged = (int64_t)p.C * ((p.OH - 1) * p.SH + p.KH) * (p.W + 2 * p.PW);
  if ((int64_t)p.OH * p.OW > kStemPix || staged > kStemLdsInput || (int64_t)p.KH * p.KW * p.C * 16 > kStemLdsW)
    return set_error(-2, "stem_conv_bn_lif_pool: image too large for the fused stem (OH*OW <= 256 and the "
                         "staged input / weights must fit in LDS); use stem_conv_bn + neuron + max-pool");
  p.spikes = reinterpret_cast<uint16_t*>(spikes);
  p.pooled = reinterpret_cast<uint16_t*>(pooled);
  p.T = d->T; p.PK = pool_k; p.PS = pool_stride; p.PP = pool_pad;
  p.np = make_neuron_params(d->neuron, d->hard_reset, d->tau, d->v_threshold, d->v_reset);
  const unsigned blocks = (unsigned)(p.N * (p.F / 16));
  if (p.KW == 7)
    hipLaunchKernelGGL((stem_conv_bn_lds_kernel<7, true>), dim3(blocks), dim3(kStemPix), 0, stream, p);
  else
    hipLaunchKernelGGL((stem_conv_bn_lds_kernel<0, true>), dim3(blocks), dim3(kStemPix), 0, stream, p);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_multistep_neuron_repeat(int32_t T, int64_t n, int32_t neuron, int32_t hard_reset,
                                                   float tau, float v_threshold, float v_reset, const float* x,
                                                   uint32_t* spikes, hipStream_t stream) {
  if (T < 1 || n < 1) return set_error(-2, "multistep_neuron_repeat: T and n must be >= 1");
  if (!x || !spikes) return set_error(-1, "multistep_neuron_repeat: null pointer");
  if (const char* why = neuron_invalid(neuron, tau)) return set_error(-2, why);
  if (n % 32 != 0) return set_error(-2, "multistep_neuron_repeat: n % 32 != 0");
  RepeatNeuronParams p{x, spikes, n, T, make_neuron_params(neuron, hard_reset, tau, v_threshold, v_reset)};
  hipLaunchKernelGGL(repeat_neuron_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_maxpool_spikes(int32_t NT, int32_t H, int32_t W, int32_t C, int32_t k, int32_t stride,
                                          int32_t pad, const uint32_t* in, uint32_t* out, hipStream_t stream) {
  if (!in || !out) return set_error(-1, "maxpool_spikes: null pointer");
  if (NT < 1 || H < 1 || W < 1 || C < 32 || C % 32 != 0 || k < 1 || stride < 1 || pad < 0 || 2 * pad >= k + 1)
    return set_error(-2, "maxpool_spikes: invalid shape (C % 32 == 0, pad < k/2 + 1)");
  PoolParams p{in, out, NT, H, W, C / 32, k, stride, pad, (H + 2 * pad - k) / stride + 1, (W + 2 * pad - k) / stride + 1};
  if (p.OH < 1 || p.OW < 1) return set_error(-2, "maxpool_spikes: empty output");
  const int64_t total = (int64_t)NT * p.OH * p.OW * p.CW;
  hipLaunchKernelGGL(maxpool_bits_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_sew_head(int32_t T, int32_t B, int32_t HW, int32_t C, int32_t planes,
                                    const uint32_t* in, const float* fc_weight, const float* fc_bias, int32_t N_out,
                                    float* out, hipStream_t stream) {
  if (!in || !fc_weight || !fc_bias || !out) return set_error(-1, "sew_head: null pointer");
  if (T < 1 || B < 1 || HW < 1 || C < 32 || C % 32 != 0 || planes < 1 || planes > kMaxPlanes || N_out < 1 ||
      (int64_t)planes * C > HEAD_MAX_PC)
    return set_error(-2, "sew_head: invalid shape (C % 32 == 0, 1 <= planes <= 5, planes * C <= 8192)");
  HeadParams p{in, fc_weight, fc_bias, out, T, B, HW, C, planes, N_out};
  // a few output slices per image, so that about 512 workgroups share the chip
  const int passes = (N_out + 4 * HEAD_OPW - 1) / (4 * HEAD_OPW);
  const int slices = std::max(1, std::min(passes, (512 + B - 1) / B));
  hipLaunchKernelGGL(sew_head_kernel, dim3((unsigned)B, (unsigned)slices), dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}
