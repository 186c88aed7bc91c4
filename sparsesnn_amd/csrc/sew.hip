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
};

constexpr int kStemLdsFloats = 16384;  // weights
constexpr int kStemLdsInput = 8192;    // staged input rows

// Workgroup = one image n and R consecutive output rows; thread = (row, ow, 16-channel
// group).  The workgroup stages the HWIO weights and the input rows its outputs read (all
// C_in channels, zero rows outside the image) in LDS, so the inner loop is LDS reads and
// FMAs only.
__global__ __launch_bounds__(256) void stem_conv_bn_lds_kernel(StemParams p, int R) {
  __shared__ float sw[kStemLdsFloats];
  __shared__ float sx[kStemLdsInput];
  // weights: float4 copies, 8 in flight per thread (p.F % 16 == 0 so nw % 4 == 0)
  const int nw4 = p.KH * p.KW * p.C * p.F / 4;
  const float4* w4src = reinterpret_cast<const float4*>(p.w);
  float4* w4dst = reinterpret_cast<float4*>(sw);
  for (int i0 = threadIdx.x; i0 < nw4; i0 += 8 * blockDim.x) {
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * blockDim.x;
      v[u] = i < nw4 ? w4src[i] : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * blockDim.x;
      if (i < nw4) w4dst[i] = v[u];
    }
  }
  const int row_blocks = (p.OH + R - 1) / R;
  const int n = blockIdx.x / row_blocks;
  const int oh0 = (blockIdx.x - n * row_blocks) * R;
  const int ih0 = oh0 * p.SH - p.PH;
  const int nrows = (R - 1) * p.SH + p.KH;
  const int nx = p.C * nrows * p.W;
  for (int i0 = threadIdx.x; i0 < nx; i0 += 8 * blockDim.x) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * blockDim.x;
      const int c = i / (nrows * p.W);
      const int rr = (i / p.W) % nrows;
      const int ih = ih0 + rr;
      v[u] = (i < nx && ih >= 0 && ih < p.H) ? p.x[(((int64_t)n * p.C + c) * p.H + ih) * p.W + i % p.W] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (i0 + u * blockDim.x < nx) sx[i0 + u * blockDim.x] = v[u];
  }
  __syncthreads();
  const int fgroups = p.F / 16;
  const int fg = threadIdx.x % fgroups;
  const int ow = (threadIdx.x / fgroups) % p.OW;
  const int rl = threadIdx.x / (fgroups * p.OW);
  const int oh = oh0 + rl;
  if (rl >= R || oh >= p.OH) return;
  float acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.f;
  for (int c = 0; c < p.C; ++c)
    for (int kh = 0; kh < p.KH; ++kh) {
      const float* xr = &sx[(c * nrows + rl * p.SH + kh) * p.W];
      for (int kw = 0; kw < p.KW; ++kw) {
        const int iw = ow * p.SW - p.PW + kw;
        if (iw < 0 || iw >= p.W) continue;
        const float xv = xr[iw];
        const float4* w4 = reinterpret_cast<const float4*>(&sw[((kh * p.KW + kw) * p.C + c) * p.F + fg * 16]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 wv = w4[q];
          acc[4 * q + 0] = __builtin_fmaf(xv, wv.x, acc[4 * q + 0]);
          acc[4 * q + 1] = __builtin_fmaf(xv, wv.y, acc[4 * q + 1]);
          acc[4 * q + 2] = __builtin_fmaf(xv, wv.z, acc[4 * q + 2]);
          acc[4 * q + 3] = __builtin_fmaf(xv, wv.w, acc[4 * q + 3]);
        }
      }
    }
  float* o = p.out + (((int64_t)n * p.OH + oh) * p.OW + ow) * p.F + fg * 16;
#pragma unroll
  for (int j = 0; j < 16; j += 4)
    *reinterpret_cast<float4*>(o + j) =
        float4{__builtin_fmaf(acc[j], p.scale[fg * 16 + j], p.bias[fg * 16 + j]),
               __builtin_fmaf(acc[j + 1], p.scale[fg * 16 + j + 1], p.bias[fg * 16 + j + 1]),
               __builtin_fmaf(acc[j + 2], p.scale[fg * 16 + j + 2], p.bias[fg * 16 + j + 2]),
               __builtin_fmaf(acc[j + 3], p.scale[fg * 16 + j + 3], p.bias[fg * 16 + j + 3])};
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
// (models/sewresnet.py:208-210).  in: integer activations as `planes` bit planes, NHWC with
// planes*C channels, (T*B, HW) positions.  One workgroup per image: the pooled features are
// exact integer sums scaled once, then each thread computes outputs o = tid, tid+256, ...
struct HeadParams {
  const uint32_t* in;
  const float* w;  // (C, N_out) fp32: the transposed nn.Linear weight (coalesced reads)
  const float* b;  // (N_out)
  float* out;      // (B, N_out)
  int T, B, HW, C, planes, N_out;
};

__global__ __launch_bounds__(256) void sew_head_kernel(HeadParams p) {
  extern __shared__ float feat[];  // C
  const int bimg = blockIdx.x;
  const int words = p.planes * p.C / 32;
  for (int c = threadIdx.x; c < p.C; c += blockDim.x) {
    int sum = 0;
    for (int t = 0; t < p.T; ++t)
      for (int s = 0; s < p.HW; ++s) {
        const uint32_t* px = p.in + ((int64_t)(t * p.B + bimg) * p.HW + s) * words;
        for (int pl = 0; pl < p.planes; ++pl) sum += (int)((px[(pl * p.C + c) >> 5] >> (c & 31)) & 1u) << pl;
      }
    // mean over HW then over T, as the reference: both are exact for the integer sums here
    feat[c] = ((float)sum / (float)p.HW) / (float)p.T;
  }
  __syncthreads();
  for (int o = threadIdx.x; o < p.N_out; o += blockDim.x) {
    float acc = 0.f;
    for (int c = 0; c < p.C; ++c) acc = __builtin_fmaf(feat[c], p.w[(int64_t)c * p.N_out + o], acc);
    p.out[(int64_t)bimg * p.N_out + o] = acc + p.b[o];
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
  const int per_row = p.OW * (p.F / 16);  // threads per output row in the LDS kernel
  const int R = per_row > 0 && per_row <= 256 ? 256 / per_row : 0;
  if (w_layout == SENGINE_WLAYOUT_HWIO && p.F % 16 == 0 && R > 0 &&
      (int64_t)p.KH * p.KW * p.C * p.F <= kStemLdsFloats &&
      (int64_t)p.C * ((R - 1) * p.SH + p.KH) * p.W <= kStemLdsInput) {
    const int64_t blocks = (int64_t)p.N * ((p.OH + R - 1) / R);
    hipLaunchKernelGGL(stem_conv_bn_lds_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p, R);
  } else if (w_layout == SENGINE_WLAYOUT_HWIO)
    hipLaunchKernelGGL(stem_conv_bn_kernel<1>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(stem_conv_bn_kernel<0>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_multistep_neuron_repeat(int32_t T, int64_t n, int32_t neuron, int32_t hard_reset,
                                                   float tau, float v_threshold, float v_reset, const float* x,
                                                   uint32_t* spikes, hipStream_t stream) {
  if (T < 1 || n < 1) return set_error(-2, "multistep_neuron_repeat: T and n must be >= 1");
  if (!x || !spikes) return set_error(-1, "multistep_neuron_repeat: null pointer");
  if (neuron != SENGINE_NEURON_LIF && neuron != SENGINE_NEURON_IF)
    return set_error(-2, "multistep_neuron_repeat: neuron must be LIF or IF");
  if (neuron == SENGINE_NEURON_LIF && !(tau > 0.f)) return set_error(-2, "multistep_neuron_repeat: tau must be > 0");
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
                                    const uint32_t* in, const float* fc_weight_t, const float* fc_bias, int32_t N_out,
                                    float* out, hipStream_t stream) {
  if (!in || !fc_weight_t || !fc_bias || !out) return set_error(-1, "sew_head: null pointer");
  if (T < 1 || B < 1 || HW < 1 || C < 32 || C % 32 != 0 || planes < 1 || planes > 3 || N_out < 1 || C > 8192)
    return set_error(-2, "sew_head: invalid shape (C % 32 == 0, C <= 8192, 1 <= planes <= 3)");
  HeadParams p{in, fc_weight_t, fc_bias, out, T, B, HW, C, planes, N_out};
  hipLaunchKernelGGL(sew_head_kernel, dim3((unsigned)B), dim3(256), (size_t)C * sizeof(float), stream, p);
  return (int)hipGetLastError();
}
