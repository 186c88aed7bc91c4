// Unfused fallback path and spike (un)packing for gfx950.
//
// dense_conv_bn_kernel mirrors the reference's decomposed Conv+BN kernels
// conv2d_bn_t4_kernel / conv1x1_bn_t4_kernel (sengine/kernels/conv2d_bn_if_t4.py:551-673):
// one GEMM over all T*B images with the BN epilogue acc*scale + bias.  It differs in
// keeping the BN output in fp32 (the reference rounds it to fp16, which is what breaks
// its fp32 parity, sengine/scripts/verify_correctness.py:4-9).  Used for convs whose
// weights are not 2:4 (sengine/optimizer.py:845-853 routes them to a dense conv + a
// standalone neuron) and for shapes the sparse kernel does not take.
//
// multistep_neuron_kernel mirrors lif_neuron_kernel / if_neuron_kernel
// (sengine/csrc/kernels.cuh:18-54): one thread per spatial element walks the T
// timesteps in order, so there is no cross-thread membrane race.  The arithmetic is
// that of the PyTorch neurons (models/neurons.py:121-146,169-184), including soft reset
// and v_reset, which the reference's native kernels ignore.
#include "common.h"
#include "internal.h"

namespace sengine {

struct DenseParams {
  const uint8_t* in;
  const half8_t* wvals;
  const float* scale;
  const float* bias;
  float* out;
  int B, C, H, W, F, KW, SH, SW, PH, PW, DH, DW, OH, OW;
  int M, nq;
  int64_t in_t_stride;
  float enc_scale;
};

// Workgroup = 4 waves = 64 output channels x 64 positions x all T (T*B images share the
// weights); the T loop sits inside the k loop so each weight fragment is reused T times.
template <int T, int IN_ENC, int PLANES>
__global__ __launch_bounds__(256) void dense_conv_bn_kernel(DenseParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int col = lane & 15;
  const int G = blockIdx.y;
  const int m = blockIdx.x * 64 + wave * 16 + col;
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

  const int chunks_per_tap = p.C >> 5;
  const half8_t* wv = p.wvals + (size_t)G * p.nq * PLANES * 4 * 64 + lane;
  for (int q = 0; q < p.nq; ++q) {
    const int tap = q / chunks_per_tap;
    const int c0 = (q - tap * chunks_per_tap) << 5;
    const int kr = tap / p.KW;
    const int ks = tap - kr * p.KW;
    const int ih = oh * p.SH - p.PH + kr * p.DH;
    const int iw = ow * p.SW - p.PW + ks * p.DW;
    const bool ok = mvalid && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W;
    const int64_t pix0 = ((int64_t)b * p.H + ih) * p.W + iw;
    half8_t av[PLANES][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int pl = 0; pl < PLANES; ++pl) av[pl][a] = wv[((size_t)(q * PLANES + pl) * 4 + a) * 64];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int64_t pix = pix0 + (int64_t)t * p.in_t_stride;
      half8_t bf = {};
      if (IN_ENC == SENGINE_ENC_BITS) {
        uint32_t x = 0;
        if (ok) x = p.in[pix * (p.C >> 3) + (c0 >> 3) + g];
        bf = expand_bits8(x);
      } else if (ok) {
        bf = *reinterpret_cast<const half8_t*>(reinterpret_cast<const _Float16*>(p.in) + pix * p.C + c0 + 8 * g);
      }
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int pl = 0; pl < PLANES; ++pl)
          acc[t][a] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[pl][a], bf, acc[t][a], 0, 0, 0);
    }
  }
  if (!mvalid) return;
  const int cob = G * 64 + g * 16;
  float sc[16], bi[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    sc[j] = p.scale[cob + j] * p.enc_scale;
    bi[j] = p.bias[cob + j];
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float* dst = p.out + ((size_t)t * p.M + m) * p.F + cob;
    float4_t o[4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[a][i] = __builtin_fmaf(acc[t][a][i], sc[4 * a + i], bi[4 * a + i]);
#pragma unroll
    for (int a = 0; a < 4; ++a) reinterpret_cast<float4_t*>(dst)[a] = o[a];
  }
}

template <int T, int IN_ENC, int PLANES>
static hipError_t launch_dense_t(const DenseParams& p, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((dense_conv_bn_kernel<T, IN_ENC, PLANES>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

template <int T>
static hipError_t launch_dense_enc(const DenseParams& p, int in_enc, int planes, dim3 grid, hipStream_t s) {
  if (in_enc == SENGINE_ENC_BITS && planes == 1) return launch_dense_t<T, SENGINE_ENC_BITS, 1>(p, grid, s);
  if (in_enc == SENGINE_ENC_BITS && planes == 2) return launch_dense_t<T, SENGINE_ENC_BITS, 2>(p, grid, s);
  if (in_enc == SENGINE_ENC_F16 && planes == 1) return launch_dense_t<T, SENGINE_ENC_F16, 1>(p, grid, s);
  if (in_enc == SENGINE_ENC_F16 && planes == 2) return launch_dense_t<T, SENGINE_ENC_F16, 2>(p, grid, s);
  return hipErrorInvalidValue;
}

struct NeuronKernelParams {
  const float* x;
  float* state;
  uint8_t* out;
  float* h_trace;
  int64_t n;
  int T;
  NeuronParams np;
};

template <int OUT_ENC>
__global__ __launch_bounds__(256) void multistep_neuron_kernel(NeuronKernelParams p) {
  const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool valid = s < p.n;
  const int lane = threadIdx.x & 63;
  float v = (valid && p.state) ? p.state[s] : 0.f;
  for (int t = 0; t < p.T; ++t) {
    const float x = valid ? p.x[(int64_t)t * p.n + s] : 0.f;
    float xf = x;
    if (p.np.neuron == SENGINE_NEURON_LIF && p.np.pow2) xf = x * p.np.rtau;  // exact
    const float h = neuron_charge(p.np, v, xf);
    const bool spike = valid && h >= p.np.vth;
    v = neuron_reset(p.np, h, spike);
    if (valid && p.h_trace) p.h_trace[(int64_t)t * p.n + s] = h;
    if (OUT_ENC == SENGINE_ENC_BITS) {
      const uint64_t mask = __ballot(spike);
      // n % 32 == 0, so a 32-lane half-wave maps to exactly one word when its first lane is valid
      if ((lane & 31) == 0 && valid)
        reinterpret_cast<uint32_t*>(p.out)[((int64_t)t * p.n + s) >> 5] = (uint32_t)(mask >> (lane & 32));
    } else if (valid) {
      reinterpret_cast<_Float16*>(p.out)[(int64_t)t * p.n + s] = spike ? (_Float16)1.0f : (_Float16)0.0f;
    }
  }
  if (valid && p.state) p.state[s] = v;
}

template <int X_ENC>
__global__ __launch_bounds__(256) void pack_spikes_kernel(const void* x, int64_t n, uint32_t* bits) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int lane = threadIdx.x & 63;
  bool on = false;
  if (e < n) {
    if (X_ENC == SENGINE_ENC_F16) on = (float)static_cast<const _Float16*>(x)[e] != 0.f;
    else on = static_cast<const float*>(x)[e] != 0.f;
  }
  const uint64_t mask = __ballot(on);
  if ((lane & 31) == 0 && e < n) bits[e >> 5] = (uint32_t)(mask >> (lane & 32));
}

template <int OUT_ENC>
__global__ __launch_bounds__(256) void unpack_spikes_kernel(const uint32_t* bits, int64_t n, void* out) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const bool on = (bits[e >> 5] >> (e & 31)) & 1u;
  if (OUT_ENC == SENGINE_ENC_F16) static_cast<_Float16*>(out)[e] = on ? (_Float16)1.0f : (_Float16)0.0f;
  else static_cast<float*>(out)[e] = on ? 1.0f : 0.0f;
}

}  // namespace sengine

using namespace sengine;

extern "C" int sengine_amd_dense_conv_bn(const sengine_conv_lif_desc* d, const void* data, const void* blob_values,
                                         const float* bn_scale, const float* bn_bias, float* out,
                                         hipStream_t stream) {
  Geometry geo;
  int rc = check_desc(d, &geo, false);
  if (rc) return rc;
  if (!data || !blob_values || !bn_scale || !bn_bias || !out) return set_error(-1, "dense_conv_bn: null pointer");
  if (d->T != 1 && d->T != 2 && d->T != 4 && d->T != 8) return set_error(-3, "dense_conv_bn: T must be 1, 2, 4 or 8");
  if (d->in_enc != SENGINE_ENC_BITS && d->in_enc != SENGINE_ENC_F16)
    return set_error(-2, "dense_conv_bn: in_enc must be BITS or F16");
  if (geo.M > (1ll << 30)) return set_error(-2, "dense_conv_bn: B*OH*OW too large");
  DenseParams p;
  p.in = static_cast<const uint8_t*>(data);
  p.wvals = static_cast<const half8_t*>(blob_values);
  p.scale = bn_scale;
  p.bias = bn_bias;
  p.out = out;
  p.B = d->B; p.C = d->C_in; p.H = d->H; p.W = d->W; p.F = d->C_out; p.KW = d->KW;
  p.SH = d->stride_h; p.SW = d->stride_w; p.PH = d->pad_h; p.PW = d->pad_w;
  p.DH = d->dil_h; p.DW = d->dil_w; p.OH = geo.OH; p.OW = geo.OW;
  p.M = (int)geo.M;
  p.nq = (int)(geo.K_red / 32);
  p.in_t_stride = (int64_t)d->B * d->H * d->W;
  p.enc_scale = d->in_enc == SENGINE_ENC_BITS ? 1.0f / kBitSpikeValue : 1.0f;
  dim3 grid((unsigned)((geo.M + 63) / 64), (unsigned)(d->C_out / 64));
  hipError_t e;
  switch (d->T) {
    case 1: e = launch_dense_enc<1>(p, d->in_enc, d->weight_planes, grid, stream); break;
    case 2: e = launch_dense_enc<2>(p, d->in_enc, d->weight_planes, grid, stream); break;
    case 4: e = launch_dense_enc<4>(p, d->in_enc, d->weight_planes, grid, stream); break;
    default: e = launch_dense_enc<8>(p, d->in_enc, d->weight_planes, grid, stream); break;
  }
  return (int)e;
}

extern "C" int sengine_amd_multistep_neuron(int32_t T, int64_t n, int32_t neuron, int32_t hard_reset, float tau,
                                            float v_threshold, float v_reset, const float* x, float* state,
                                            int32_t out_enc, void* spikes, float* h_trace, hipStream_t stream) {
  if (T < 1 || n < 1) return set_error(-2, "multistep_neuron: T and n must be >= 1");
  if (!x || !spikes) return set_error(-1, "multistep_neuron: null pointer");
  if (const char* why = neuron_invalid(neuron, tau)) return set_error(-2, why);
  if (out_enc == SENGINE_ENC_BITS && n % 32 != 0) return set_error(-2, "multistep_neuron: bit output needs n % 32 == 0");
  if (out_enc != SENGINE_ENC_BITS && out_enc != SENGINE_ENC_F16)
    return set_error(-2, "multistep_neuron: out_enc must be BITS or F16");
  NeuronKernelParams p{x, state, static_cast<uint8_t*>(spikes), h_trace, n, T,
                       make_neuron_params(neuron, hard_reset, tau, v_threshold, v_reset)};
  dim3 grid((unsigned)((n + 255) / 256));
  if (out_enc == SENGINE_ENC_BITS)
    hipLaunchKernelGGL(multistep_neuron_kernel<SENGINE_ENC_BITS>, grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(multistep_neuron_kernel<SENGINE_ENC_F16>, grid, dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_pack_spikes(const void* x, int32_t x_enc, int64_t n_pos, int32_t C, uint32_t* bits,
                                       hipStream_t stream) {
  if (!x || !bits) return set_error(-1, "pack_spikes: null pointer");
  if (n_pos < 0 || C < 1 || C % 32 != 0) return set_error(-2, "pack_spikes: need C % 32 == 0");
  const int64_t n = n_pos * C;
  if (n == 0) return 0;
  dim3 grid((unsigned)((n + 255) / 256));
  if (x_enc == SENGINE_ENC_F16)
    hipLaunchKernelGGL(pack_spikes_kernel<SENGINE_ENC_F16>, grid, dim3(256), 0, stream, x, n, bits);
  else if (x_enc == SENGINE_ENC_F32)
    hipLaunchKernelGGL(pack_spikes_kernel<SENGINE_ENC_F32>, grid, dim3(256), 0, stream, x, n, bits);
  else
    return set_error(-2, "pack_spikes: x_enc must be F16 or F32");
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_unpack_spikes(const uint32_t* bits, int64_t n_pos, int32_t C, void* out, int32_t out_enc,
                                         hipStream_t stream) {
  if (!bits || !out) return set_error(-1, "unpack_spikes: null pointer");
  if (n_pos < 0 || C < 1 || C % 32 != 0) return set_error(-2, "unpack_spikes: need C % 32 == 0");
  const int64_t n = n_pos * C;
  if (n == 0) return 0;
  dim3 grid((unsigned)((n + 255) / 256));
  if (out_enc == SENGINE_ENC_F16)
    hipLaunchKernelGGL(unpack_spikes_kernel<SENGINE_ENC_F16>, grid, dim3(256), 0, stream, bits, n, out);
  else if (out_enc == SENGINE_ENC_F32)
    hipLaunchKernelGGL(unpack_spikes_kernel<SENGINE_ENC_F32>, grid, dim3(256), 0, stream, bits, n, out);
  else
    return set_error(-2, "unpack_spikes: out_enc must be F16 or F32");
  return (int)hipGetLastError();
}
