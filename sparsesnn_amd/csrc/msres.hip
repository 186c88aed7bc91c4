// Real-valued 1x1 convolution + folded BN: the shortcut of an MS-ResNet block, whose input
// is the block's real-valued (membrane-shortcut) stream rather than spikes
// (BasicBlock18.shortcut = TDBNContainer(Conv2d 1x1 / stride s, BatchNorm3d),
// models/msresnet.py:113-118,111; TDBNContainer.forward :79-87).  The spike convolutions
// of the block run on the fused sparse kernels; this one multiplies fp32 activations, so it
// is a plain fp32 GEMM over the strided pixels on the fp32 matrix cores:
//   out[(t, b, oh, ow), f] = (sum_c x[(t, b, oh*S, ow*S), c] * w[c, f]) * scale[f] + bias[f]
// fp32 throughout; the matrix cores sum four products per step, so the order of the terms
// differs from a sequential sum (results agree to fp32 rounding).  When the
// input carries one timestep and the output T (the stem output that the reference repeats
// over T before the first block, models/msresnet.py:146-150), each value is computed once
// and stored T times.
#include "common.h"
#include "internal.h"

namespace sengine {

struct RealConvParams {
  const float* x;      // NHWC fp32 (N, H, W, C)
  const float* w;      // HWIO (C, F) or OIHW (F, C) fp32
  const float* scale;  // folded BN
  const float* bias;
  float* out;          // NHWC fp32 (reps * N, OH, OW, F)
  int N, C, H, W, F, S, OH, OW, reps, hwio;
  int64_t M;           // N * OH * OW output positions per repetition
};

constexpr int kRcPos = 64;  // positions per workgroup
constexpr int kRcCh = 64;   // output channels per workgroup
constexpr int kRcK = 16;    // reduction chunk staged in LDS

// Workgroup = 64 positions x 64 channels, 256 threads.  Per 16-channel reduction chunk the
// input pixels (transposed, c-major) and the weights are staged in LDS; wave w then computes
// positions 16w..16w+15 x the 64 channels on the fp32 matrix cores (v_mfma_f32_16x16x4_f32,
// four 16-channel tiles, 4 taps of the reduction per instruction): lane l feeds weight
// (tap 4s + l/16, channel l % 16 of the tile) and input (same tap, position l % 16) and ends
// holding channels 4 (l/16)..4 (l/16) + 3 of each tile for position l % 16.
__global__ __launch_bounds__(256) void real_conv1x1_bn_kernel(RealConvParams p) {
  __shared__ float xs[kRcK][kRcPos + 4];
  __shared__ float ws[kRcK][kRcCh + 4];
  __shared__ __align__(16) float sO[kRcPos][kRcCh + 4];  // output tile, wave w: rows 16w..16w+15
  const int tid = threadIdx.x;
  const int64_t m0 = (int64_t)blockIdx.x * kRcPos;
  const int f0 = blockIdx.y * kRcCh;

  // staging identity: position lp = tid / 4, channels 4*(tid % 4) .. +3 of the chunk
  const int lp = tid >> 2, lq = tid & 3;
  const int64_t ms = m0 + lp;
  const bool svalid = ms < p.M;
  const float* xrow = p.x;
  if (svalid) {
    const int64_t ohw = (int64_t)p.OH * p.OW;
    const int64_t n = ms / ohw;
    const int r = (int)(ms - n * ohw);
    const int oh = r / p.OW, ow = r - (r / p.OW) * p.OW;
    xrow = p.x + ((n * p.H + (int64_t)oh * p.S) * p.W + (int64_t)ow * p.S) * p.C;
  }
  const int wk = tid >> 4, wf = (tid & 15) * 4;  // weight staging: row wk, channels wf..wf+3
  const int wave = tid >> 6, lane = tid & 63, q = lane >> 4, j = lane & 15;

  float4_t acc[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) acc[nb] = float4_t{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < p.C; k0 += kRcK) {
    const float4 xv = svalid ? *reinterpret_cast<const float4*>(xrow + k0 + 4 * lq) : float4{0.f, 0.f, 0.f, 0.f};
    float4 wv;
    if (p.hwio) {
      wv = *reinterpret_cast<const float4*>(p.w + (int64_t)(k0 + wk) * p.F + f0 + wf);
    } else {
      const float* wc = p.w + (int64_t)(f0 + wf) * p.C + k0 + wk;
      wv = float4{wc[0], wc[p.C], wc[2 * p.C], wc[3 * p.C]};
    }
    __syncthreads();  // previous chunk fully consumed
    xs[4 * lq + 0][lp] = xv.x;
    xs[4 * lq + 1][lp] = xv.y;
    xs[4 * lq + 2][lp] = xv.z;
    xs[4 * lq + 3][lp] = xv.w;
    *reinterpret_cast<float4*>(&ws[wk][wf]) = wv;
    __syncthreads();
#pragma unroll
    for (int s = 0; s < kRcK / 4; ++s) {
      const float xb = xs[4 * s + q][16 * wave + j];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(ws[4 * s + q][16 * nb + j], xb, acc[nb], 0, 0, 0);
    }
  }

  // The wave's 16 x 64 tile goes through LDS (its own rows only: no barrier) so that each
  // store instruction writes four whole 256-byte position rows.
  float* so = &sO[16 * wave][0];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
    *reinterpret_cast<float4_t*>(so + j * (kRcCh + 4) + 16 * nb + 4 * q) = acc[nb];
  const int f = f0 + 4 * j;
  const float4 sc = *reinterpret_cast<const float4*>(p.scale + f);
  const float4 bi = *reinterpret_cast<const float4*>(p.bias + f);
  const int64_t rep_stride = p.M * p.F;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * i + q;  // position 16 wave + row, channels 4j..4j+3
    const int64_t m = m0 + 16 * wave + row;
    const float4_t a = *reinterpret_cast<const float4_t*>(so + row * (kRcCh + 4) + 4 * j);
    if (m >= p.M) continue;
    const float4 o{__builtin_fmaf(a[0], sc.x, bi.x), __builtin_fmaf(a[1], sc.y, bi.y),
                   __builtin_fmaf(a[2], sc.z, bi.z), __builtin_fmaf(a[3], sc.w, bi.w)};
    float* dst = p.out + m * p.F + f;
    for (int r = 0; r < p.reps; ++r) *reinterpret_cast<float4*>(dst + r * rep_stride) = o;
  }
}

}  // namespace sengine

using namespace sengine;

extern "C" int sengine_amd_real_conv_bn(const sengine_conv_lif_desc* d, const float* x, int32_t in_T,
                                        const float* weight, int32_t w_layout, const float* bn_scale,
                                        const float* bn_bias, float* out, hipStream_t stream) {
  if (!d || !x || !weight || !bn_scale || !bn_bias || !out) return set_error(-1, "real_conv_bn: null pointer");
  if (w_layout != SENGINE_WLAYOUT_OIHW && w_layout != SENGINE_WLAYOUT_HWIO)
    return set_error(-2, "real_conv_bn: w_layout must be OIHW or HWIO");
  if (d->T < 1 || d->B < 1 || d->H < 1 || d->W < 1 || d->C_in < 1 || d->C_out < 1)
    return set_error(-2, "real_conv_bn: invalid shape fields");
  if (d->KH != 1 || d->KW != 1 || d->pad_h != 0 || d->pad_w != 0 || d->dil_h != 1 || d->dil_w != 1 ||
      d->stride_h < 1 || d->stride_h != d->stride_w)
    return set_error(-2, "real_conv_bn: 1x1 kernel, no padding, equal strides only");
  if (d->C_in % kRcK != 0 || d->C_out % kRcCh != 0)
    return set_error(-2, "real_conv_bn: C_in % 16 == 0 and C_out % 64 == 0 required");
  if (in_T != 1 && in_T != d->T) return set_error(-2, "real_conv_bn: in_T must be 1 (repeated over T) or T");
  RealConvParams p{};
  p.x = x; p.w = weight; p.scale = bn_scale; p.bias = bn_bias; p.out = out;
  p.N = in_T * d->B; p.C = d->C_in; p.H = d->H; p.W = d->W; p.F = d->C_out; p.S = d->stride_h;
  p.OH = (d->H - 1) / d->stride_h + 1;
  p.OW = (d->W - 1) / d->stride_w + 1;
  p.reps = in_T == 1 ? d->T : 1;
  p.hwio = w_layout == SENGINE_WLAYOUT_HWIO;
  p.M = (int64_t)p.N * p.OH * p.OW;
  const int64_t gx = (p.M + kRcPos - 1) / kRcPos;
  if (gx > 0x7fffffff) return set_error(-2, "real_conv_bn: too many positions");
  hipLaunchKernelGGL(real_conv1x1_bn_kernel, dim3((unsigned)gx, (unsigned)(p.F / kRcCh)), dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}
