// Weight preparation kernels: 2:4 compressor (sparse blob) and dense packer.
//
// The reference keeps conv weights dense (KH, KW, C_in, C_out) on the device
// (sengine/cuda_graph_runtime.py:233-235) and only validates the 2:4 pattern
// (sengine/optimizer.py:499-553); the compressed format below is specific to the
// gfx950 SMFMAC operand layout (see common.h) and is produced once per node at
// build time.
//
// Sparse blob, per 64-output-channel group G and 64-wide reduction chunk q
// (K_red ordered (kh, kw, c_in)):
//   values[G][q][plane][tile a][lane][8 x fp16]   (16 B per lane, one A operand)
//   meta  [G][q][lane][tile a] u32                (low 16 bits: 8 x 2-bit positions; a lane's
//                                                  four tiles in one 16-byte load)
// Row permutation: A tile a, row r <-> output channel 64G + 16*(r/4) + 4a + r%4, so the
// accumulator of lane group g holds channels 16g..16g+15 (see fused_sparse.hip).
// Planes: plane 0 = fp16(w); plane 1 (optional) = fp16(w - plane0), which makes the
// fp16 pair carry ~22 significant bits of an fp32 weight.
#include "common.h"
#include "internal.h"

namespace sengine {

__device__ __forceinline__ float load_weight(const void* w, int w_enc, int w_layout, int co, int ci, int kh, int kw,
                                             int C_out, int C_in, int KH, int KW) {
  size_t idx;
  if (w_layout == SENGINE_WLAYOUT_OIHW)
    idx = (((size_t)co * C_in + ci) * KH + kh) * KW + kw;
  else
    idx = (((size_t)kh * KW + kw) * C_in + ci) * C_out + co;
  if (w_enc == SENGINE_ENC_F16) return (float)static_cast<const _Float16*>(w)[idx];
  return static_cast<const float*>(w)[idx];
}

struct WeightParams {
  const void* w;
  int w_enc, w_layout;
  int C_out, C_in, KH, KW;
  int nq;
  int planes;
  // flat layout (sparse blob only): rows (opix, c_out), reduction (ipix, c_in)
  int flat, W, OW, SH, SW, PH, PW, DH, DW;
  int rows;  // blob rows: C_out, or OH*OW*C_out in the flat layout
  int tail;  // 3x3 paired-tail form: the last 64-channel chunk holds 32 real channels
};

// Flat layout: the conv tap that input pixel ipix contributes to output pixel opix
// through, or false when it falls outside the kernel.
__device__ __forceinline__ bool flat_tap(const WeightParams& p, int opix, int ipix, int& kh, int& kw) {
  const int oh = opix / p.OW, ow = opix - (opix / p.OW) * p.OW;
  const int ih = ipix / p.W, iw = ipix - (ipix / p.W) * p.W;
  const int dh = ih - oh * p.SH + p.PH, dw = iw - ow * p.SW + p.PW;
  if (dh < 0 || dw < 0 || dh % p.DH != 0 || dw % p.DW != 0) return false;
  kh = dh / p.DH;
  kw = dw / p.DW;
  return kh < p.KH && kw < p.KW;
}

// Zero test of validate_2_4_pattern (sengine/optimizer.py:522): |w| < 1e-10.
__device__ __forceinline__ bool is_kept(float x) { return fabsf(x) >= 1e-10f; }

__global__ __launch_bounds__(256) void compress_2_4_kernel(WeightParams p, half8_t* vals, uint32_t* meta,
                                                           int32_t* violations) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)(p.rows / 64) * p.nq * 4 * 64;
  if (tid >= total) return;
  const int lane = (int)(tid & 63);
  const int a = (int)((tid >> 6) & 3);
  const int64_t gq = tid >> 8;  // G * nq + q
  const int q = (int)(gq % p.nq);
  const int G = (int)(gq / p.nq);
  const int r = lane & 15;
  const int row = G * 64 + 16 * (r >> 2) + 4 * a + (r & 3);
  const int kbase = q * 64 + 16 * (lane >> 4);
  int tap = kbase / p.C_in;  // flat layout: the input pixel
  int cin0 = kbase - tap * p.C_in;
  bool inside = true;
  if (p.tail) {
    // 9 * nfull full chunks in (tap, chunk) order, then 5 chunks pairing taps 2i, 2i + 1 over
    // the last chunk's 32 real channels: lane groups 0, 1 the first tap, 2, 3 the second
    const int nfull = p.C_in / 64 - 1, g = lane >> 4;
    if (q < 9 * nfull) {
      tap = q / nfull;
      cin0 = (q - tap * nfull) * 64 + 16 * g;
    } else {
      tap = 2 * (q - 9 * nfull) + (g >> 1);
      cin0 = nfull * 64 + 16 * (g & 1);
      if (tap > 8) inside = false, tap = 8;  // tap 8 has no partner: zero weights
    }
  }
  int co = row, kh = tap / p.KW, kw = tap - (tap / p.KW) * p.KW;
  if (p.flat) {
    const int opix = row / p.C_out;
    co = row - opix * p.C_out;
    inside = flat_tap(p, opix, tap, kh, kw);
  }

  float kept[8];
  uint32_t bits = 0;
#pragma unroll
  for (int gi = 0; gi < 4; ++gi) {
    float w4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w4[e] = inside ? load_weight(p.w, p.w_enc, p.w_layout, co, cin0 + 4 * gi + e, kh, kw, p.C_out, p.C_in, p.KH,
                                   p.KW)
                     : 0.f;
    int pos[2] = {-1, -1};
    int n = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (is_kept(w4[e])) {
        if (n < 2) pos[n] = e;
        ++n;
      }
    // pad with the lowest unused positions (value 0) so every group has two slots
    for (int e = 0; e < 4 && (pos[0] < 0 || pos[1] < 0); ++e) {
      if (e == pos[0] || e == pos[1]) continue;
      if (pos[0] < 0) pos[0] = e;
      else pos[1] = e;
    }
    if (pos[0] > pos[1]) { const int tmp = pos[0]; pos[0] = pos[1]; pos[1] = tmp; }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float x = w4[pos[s]];
      kept[2 * gi + s] = is_kept(x) ? x : 0.f;
      bits |= (uint32_t)pos[s] << (2 * (2 * gi + s));
    }
    if (violations && inside) {  // flat layout: every copy of a group writes the same value
      const int64_t gid = (((int64_t)co * p.KH + kh) * p.KW + kw) * (p.C_in / 4) + (cin0 / 4) + gi;
      violations[gid] = n > 2 ? 1 : 0;
    }
  }
  half8_t v0, v1;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const _Float16 hi = (_Float16)kept[j];
    v0[j] = hi;
    v1[j] = (_Float16)(kept[j] - (float)hi);
  }
  const size_t base = ((size_t)gq * p.planes) * 4 * 64 + (size_t)a * 64 + lane;
  vals[base] = v0;
  if (p.planes == 2) vals[base + 4 * 64] = v1;
  meta[(size_t)gq * 4 * 64 + (size_t)lane * 4 + a] = bits;
}

// Paired-tail form: the last 32 input channels are not in the blob; a group of four of them
// holding any entry with |w| >= 1e-10 is reported as a violation.
__global__ __launch_bounds__(256) void tail_zero_check_kernel(WeightParams p, int32_t* violations) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.C_out * 9 * 8;  // (c_out, tap, group of the last 32 channels)
  if (tid >= total) return;
  const int gi = (int)(tid & 7);
  const int tap = (int)((tid >> 3) % 9);
  const int co = (int)(tid / 72);
  const int kh = tap / 3, kw = tap - (tap / 3) * 3;
  const int c0 = p.C_in - 32 + 4 * gi;
  int n = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    n += is_kept(load_weight(p.w, p.w_enc, p.w_layout, co, c0 + e, kh, kw, p.C_out, p.C_in, 3, 3)) ? 1 : 0;
  violations[(((int64_t)co * 3 + kh) * 3 + kw) * (p.C_in / 4) + c0 / 4] = n > 0 ? 1 : 0;
}

// Dense blob: values[G][q32][plane][tile a][lane][8 x fp16], A operand of
// v_mfma_f32_16x16x32_f16 with the same row permutation as the sparse blob.
__global__ __launch_bounds__(256) void pack_dense_kernel(WeightParams p, half8_t* vals) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)(p.C_out / 64) * p.nq * 4 * 64;
  if (tid >= total) return;
  const int lane = (int)(tid & 63);
  const int a = (int)((tid >> 6) & 3);
  const int64_t gq = tid >> 8;
  const int q = (int)(gq % p.nq);
  const int G = (int)(gq / p.nq);
  const int r = lane & 15;
  const int co = G * 64 + 16 * (r >> 2) + 4 * a + (r & 3);
  const int kbase = q * 32 + 8 * (lane >> 4);
  const int tap = kbase / p.C_in;
  const int cin0 = kbase - tap * p.C_in;
  const int kh = tap / p.KW;
  const int kw = tap - kh * p.KW;
  half8_t v0, v1;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float x = load_weight(p.w, p.w_enc, p.w_layout, co, cin0 + j, kh, kw, p.C_out, p.C_in, p.KH, p.KW);
    const _Float16 hi = (_Float16)x;
    v0[j] = hi;
    v1[j] = (_Float16)(x - (float)hi);
  }
  const size_t base = ((size_t)gq * p.planes) * 4 * 64 + (size_t)a * 64 + lane;
  vals[base] = v0;
  if (p.planes == 2) vals[base + 4 * 64] = v1;
}

}  // namespace sengine

using namespace sengine;

extern "C" int sengine_amd_compress_2_4(const sengine_conv_lif_desc* d, const void* weight, int32_t w_enc,
                                        int32_t w_layout, void* blob_values, void* blob_meta,
                                        int32_t* violations, hipStream_t stream) {
  Geometry geo;
  int rc = check_desc(d, &geo, true);
  if (rc) return rc;
  if (!weight || !blob_values || !blob_meta) return set_error(-1, "compress_2_4: null pointer");
  if (w_enc != SENGINE_ENC_F32 && w_enc != SENGINE_ENC_F16)
    return set_error(-2, "compress_2_4: weight encoding must be F32 or F16");
  if (w_layout != SENGINE_WLAYOUT_OIHW && w_layout != SENGINE_WLAYOUT_HWIO)
    return set_error(-2, "compress_2_4: unknown weight layout");
  const bool flat = flat_layout(d, geo);
  WeightParams p{weight, w_enc, w_layout, d->C_out, d->C_in, d->KH, d->KW, (int)(geo.K_red / 64), d->weight_planes,
                 flat ? 1 : 0, d->W, geo.OW, d->stride_h, d->stride_w, d->pad_h, d->pad_w, d->dil_h, d->dil_w,
                 d->C_out};
  if (flat) {
    p.nq = (int)((int64_t)d->H * d->W * d->C_in / 64);
    p.rows = geo.OH * geo.OW * d->C_out;
  }
  const int64_t total = (int64_t)(p.rows / 64) * p.nq * 256;
  hipLaunchKernelGGL(compress_2_4_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, p,
                     static_cast<half8_t*>(blob_values), static_cast<uint32_t*>(blob_meta), violations);
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_compress_2_4_tail(const sengine_conv_lif_desc* d, const void* weight, int32_t w_enc,
                                             int32_t w_layout, void* blob_values, void* blob_meta,
                                             int32_t* violations, hipStream_t stream) {
  Geometry geo;
  int rc = check_desc(d, &geo, true);
  if (rc) return rc;
  if ((rc = check_tail_desc(d, "compress_2_4_tail"))) return rc;
  if (!weight || !blob_values || !blob_meta) return set_error(-1, "compress_2_4_tail: null pointer");
  if (w_enc != SENGINE_ENC_F32 && w_enc != SENGINE_ENC_F16)
    return set_error(-2, "compress_2_4_tail: weight encoding must be F32 or F16");
  if (w_layout != SENGINE_WLAYOUT_OIHW && w_layout != SENGINE_WLAYOUT_HWIO)
    return set_error(-2, "compress_2_4_tail: unknown weight layout");
  WeightParams p{weight, w_enc, w_layout, d->C_out, d->C_in, 3, 3, tail_chunks(d), d->weight_planes,
                 0, d->W, geo.OW, 1, 1, 1, 1, 1, 1, d->C_out, 1};
  const int64_t total = (int64_t)(p.rows / 64) * p.nq * 256;
  hipLaunchKernelGGL(compress_2_4_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, p,
                     static_cast<half8_t*>(blob_values), static_cast<uint32_t*>(blob_meta), violations);
  if (violations) {
    const int64_t nz = (int64_t)d->C_out * 72;
    hipLaunchKernelGGL(tail_zero_check_kernel, dim3((unsigned)((nz + 255) / 256)), dim3(256), 0, stream, p,
                       violations);
  }
  return (int)hipGetLastError();
}

extern "C" int sengine_amd_pack_dense_weights(const sengine_conv_lif_desc* d, const void* weight, int32_t w_enc,
                                              int32_t w_layout, void* blob_values, hipStream_t stream) {
  Geometry geo;
  int rc = check_desc(d, &geo, false);
  if (rc) return rc;
  if (!weight || !blob_values) return set_error(-1, "pack_dense_weights: null pointer");
  if (w_enc != SENGINE_ENC_F32 && w_enc != SENGINE_ENC_F16)
    return set_error(-2, "pack_dense_weights: weight encoding must be F32 or F16");
  if (w_layout != SENGINE_WLAYOUT_OIHW && w_layout != SENGINE_WLAYOUT_HWIO)
    return set_error(-2, "pack_dense_weights: unknown weight layout");
  WeightParams p{weight, w_enc, w_layout, d->C_out, d->C_in, d->KH, d->KW, (int)(geo.K_red / 32), d->weight_planes,
                 0, 0, 0, 0, 0, 0, 0, 0, 0, d->C_out};
  const int64_t total = (int64_t)(d->C_out / 64) * p.nq * 256;
  hipLaunchKernelGGL(pack_dense_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, p,
                     static_cast<half8_t*>(blob_values));
  return (int)hipGetLastError();
}
