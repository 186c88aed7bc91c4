// On-box peak calibration for the roofline (the role of the reference's
// sengine/tuning/hw_calibrate.py:17-134, which times a large memcpy and a dense fp16 GEMM).
//
//  * calib_smfmac_kernel: every wave issues back-to-back v_smfmac_f32_16x16x64_f16 on eight
//    independent accumulators with register operands (no memory traffic), so the launch
//    measures the sparse matrix-core issue rate the fused kernels are priced against.
//  * calib_copy_kernel: a 16-byte-per-lane streaming copy over a caller buffer (read + write),
//    the HBM bound of the memory-bound layers; calib_copy_nt_kernel the same copy with
//    non-temporal loads and stores (no cache allocation), calib_read_kernel a read-only
//    stream folded into one word per thread (the read ceiling with no write traffic).
#include "common.h"
#include "internal.h"

namespace sengine {

__global__ __launch_bounds__(256) void calib_smfmac_kernel(int iters, float* __restrict__ sink) {
  const int lane = (int)(threadIdx.x & 63);
  // lane-dependent operands so nothing folds; values stay small (sums stay finite)
  half8_t a;
  half16_t b;
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = (_Float16)(0.001f * (float)((lane + j) & 7));
#pragma unroll
  for (int j = 0; j < 16; ++j) b[j] = (_Float16)(0.001f * (float)((lane * 3 + j) & 7));
  const int idx = (int)0x4E4E4E4Eu;  // every 4-group keeps positions {2, 3} and {0, 1}
  float4_t acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = __builtin_amdgcn_smfmac_f32_16x16x64_f16(a, b, acc[k], idx, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) s += acc[k][0] + acc[k][1] + acc[k][2] + acc[k][3];
  sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

__global__ __launch_bounds__(256) void calib_copy_kernel(const u32x4_t* __restrict__ src, u32x4_t* __restrict__ dst,
                                                         int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

// Four 16-byte pieces in flight per lane per trip (strided by the grid), the rest one by one.
__global__ __launch_bounds__(256) void calib_copy_nt_kernel(const u32x4_t* __restrict__ src,
                                                            u32x4_t* __restrict__ dst, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    u32x4_t v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = __builtin_nontemporal_load(src + i + k * stride);
#pragma unroll
    for (int k = 0; k < 4; ++k) __builtin_nontemporal_store(v[k], dst + i + k * stride);
  }
  for (; i < n16; i += stride) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

__global__ __launch_bounds__(256) void calib_read_kernel(const u32x4_t* __restrict__ src, uint32_t* __restrict__ sink,
                                                         int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t s = 0;
  int64_t i = tid;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    u32x4_t v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = src[i + k * stride];
#pragma unroll
    for (int k = 0; k < 4; ++k) s ^= v[k][0] ^ v[k][1] ^ v[k][2] ^ v[k][3];
  }
  for (; i < n16; i += stride) {
    const u32x4_t v = src[i];
    s ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  sink[tid] = s;
}

}  // namespace sengine

using namespace sengine;

extern "C" int sengine_amd_calibrate_smfmac(int32_t blocks, int32_t iters, float* sink, hipStream_t stream) {
  if (blocks <= 0 || iters <= 0) return set_error(-2, "calibrate_smfmac: blocks and iters must be positive");
  if (!sink) return set_error(-1, "calibrate_smfmac: null sink");
  hipLaunchKernelGGL(calib_smfmac_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, (int)iters, sink);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_calibrate_copy(const void* src, void* dst, int64_t bytes, hipStream_t stream) {
  if (!src || !dst) return set_error(-1, "calibrate_copy: null buffer");
  if (bytes <= 0 || bytes % 16 != 0) return set_error(-2, "calibrate_copy: bytes must be a positive multiple of 16");
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15)
    return set_error(-2, "calibrate_copy: buffers must be 16-byte aligned");
  const int64_t n16 = bytes / 16;
  // a few waves per SIMD over 256 CUs; every lane moves 16 bytes per trip
  const int64_t want = (n16 + 255) / 256;
  const unsigned grid = (unsigned)(want < 4096 ? want : 4096);
  hipLaunchKernelGGL(calib_copy_kernel, dim3(grid), dim3(256), 0, stream, static_cast<const u32x4_t*>(src),
                     static_cast<u32x4_t*>(dst), n16);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_calibrate_stream(const void* src, void* dst, int64_t bytes, int32_t mode,
                                            hipStream_t stream) {
  if (!src || !dst) return set_error(-1, "calibrate_stream: null buffer");
  if (mode < 0 || mode > 2) return set_error(-2, "calibrate_stream: mode must be 0 (copy), 1 (non-temporal copy) or 2 (read)");
  if (bytes <= 0 || bytes % 16 != 0) return set_error(-2, "calibrate_stream: bytes must be a positive multiple of 16");
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15)
    return set_error(-2, "calibrate_stream: buffers must be 16-byte aligned");
  if (mode == 0) return sengine_amd_calibrate_copy(src, dst, bytes, stream);
  const int64_t n16 = bytes / 16;
  const int64_t want = (n16 + 255) / 256;
  const unsigned grid = (unsigned)(want < 4096 ? want : 4096);
  if (mode == 1)
    hipLaunchKernelGGL(calib_copy_nt_kernel, dim3(grid), dim3(256), 0, stream, static_cast<const u32x4_t*>(src),
                       static_cast<u32x4_t*>(dst), n16);
  else  // one 32-bit word per thread: grid * 256 * 4 <= bytes / 4 <= the buffer
    hipLaunchKernelGGL(calib_read_kernel, dim3(grid), dim3(256), 0, stream, static_cast<const u32x4_t*>(src),
                       static_cast<uint32_t*>(dst), n16);
  return (int)hipGetLastError();
}
