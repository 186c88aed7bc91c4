// The reference runtime's weight tensor behind the fused call (host side).
//
// The reference's per-node call() receives the runtime's fp16 weight in (KH, KW, C_in, C_out)
// layout (sengine/cuda_graph_runtime.py:233-235, passed by sengine/csrc/cpp_executor.cu:
// 909-913) and reads it on every call.  This build's kernels read a 2:4 blob (SMFMAC-ordered
// values + metadata).  The entries below keep one blob per (device, weight pointer,
// descriptor): built on the first call outside stream capture (the reference executor runs
// every node eagerly three times before it captures, cpp_executor.cu:1270-1276) and reused by
// later calls.  A cached blob is only as good as the bytes it was built from -- the caller may
// update the weight in place, or free it and let its allocator hand the address to a different
// weight -- so every call outside stream capture re-reads the whole weight into a 64-bit
// fingerprint and rebuilds the blob (in place: captured graphs keep pointing at it) when the
// fingerprint differs from the one recorded at the last build.  Calls inside a capture cannot
// synchronise and use the blob as of the last eager call.  A first call inside a capture is
// refused (it would have to allocate).
#include <algorithm>
#include <mutex>
#include <vector>

#include "common.h"
#include "internal.h"

namespace {

constexpr int kFpThreads = 256;
constexpr int kFpMaxBlocks = 512;

// splitmix64's output function (a bijection on 64-bit words; Steele, Lea and Flood, "Fast
// splittable pseudorandom number generators", OOPSLA 2014).
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// Fingerprint of n 32-bit words: the sum (mod 2^64) over i of mix64(i << 32 | w[i]).  Every
// (position, value) pair maps to a distinct mixed word, so changing any single word always
// changes the sum; the sum is independent of the order the threads add in.
__global__ __launch_bounds__(kFpThreads) void weight_fingerprint_kernel(const uint32_t* __restrict__ w, int64_t n,
                                                                        unsigned long long* __restrict__ out) {
  __shared__ uint64_t part[kFpThreads];
  uint64_t acc = 0;
  for (int64_t i = (int64_t)blockIdx.x * kFpThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kFpThreads)
    acc += mix64(((uint64_t)i << 32) | (uint64_t)w[i]);
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int s = kFpThreads / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) part[threadIdx.x] += part[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) atomicAdd(out, (unsigned long long)part[0]);
}

struct BlobEntry {
  int dev;
  const void* weight;
  sengine_conv_lif_desc desc;
  int32_t w_enc, w_layout;
  void* blob;            // values | metadata | 256 bytes holding the fingerprint accumulator
  size_t value_bytes;
  size_t fp_offset;      // byte offset of the fingerprint accumulator in `blob`
  uint64_t fingerprint;  // of the weight bytes the blob was last built from
  bool valid;            // false: the last build found a weight that is not 2:4
};

std::mutex g_mu;
std::vector<BlobEntry> g_blobs;

bool same_desc(const sengine_conv_lif_desc& a, const sengine_conv_lif_desc& b) {
  // the weight blob depends on the geometry and weight planes only; in_enc / out_enc and the
  // neuron parameters may differ between calls sharing a blob
  return a.C_out == b.C_out && a.C_in == b.C_in && a.KH == b.KH && a.KW == b.KW && a.H == b.H && a.W == b.W &&
         a.stride_h == b.stride_h && a.stride_w == b.stride_w && a.pad_h == b.pad_h && a.pad_w == b.pad_w &&
         a.dil_h == b.dil_h && a.dil_w == b.dil_w && a.weight_planes == b.weight_planes && a.T == b.T && a.B == b.B;
}

BlobEntry* find_blob(int dev, const void* w, const sengine_conv_lif_desc* d, int32_t w_enc, int32_t w_layout) {
  for (BlobEntry& e : g_blobs)
    if (e.dev == dev && e.weight == w && e.w_enc == w_enc && e.w_layout == w_layout && same_desc(e.desc, *d)) return &e;
  return nullptr;
}

// Bytes of the raw weight (KH*KW*C_in*C_out elements of w_enc); 0 for an unknown encoding.
size_t weight_bytes(const sengine_conv_lif_desc* d, int32_t w_enc) {
  const size_t n = (size_t)d->KH * d->KW * d->C_in * d->C_out;
  if (w_enc == SENGINE_ENC_F16) return n * 2;
  if (w_enc == SENGINE_ENC_F32) return n * 4;
  return 0;
}

// Queues the fingerprint of the weight into acc (cleared first) on `stream`.
hipError_t queue_fingerprint(const void* weight, size_t nbytes, unsigned long long* acc, hipStream_t stream) {
  hipError_t e = hipMemsetAsync(acc, 0, sizeof(*acc), stream);  // never captured: eager calls only
  if (e != hipSuccess) return e;
  const int64_t n = (int64_t)(nbytes / 4);  // C_in % 64 == 0 on the sparse path: whole words
  const int blocks = (int)std::min<int64_t>(kFpMaxBlocks, std::max<int64_t>(1, (n + kFpThreads - 1) / kFpThreads));
  hipLaunchKernelGGL(weight_fingerprint_kernel, dim3(blocks), dim3(kFpThreads), 0, stream,
                     static_cast<const uint32_t*>(weight), n, acc);
  return hipGetLastError();
}

// (Re)builds entry e's blob from the weight: compression into the existing blob, the 2:4 check
// and the fingerprint, with one synchronisation.  Returns 0, -5 (not 2:4: e.valid = false) or
// a positive hipError_t.
int build_blob(BlobEntry& e, hipStream_t stream) {
  const int64_t ngroups = sengine_amd_num_groups(&e.desc);
  if (ngroups <= 0) return sengine::set_error(-2, "prepare_weight: invalid descriptor");
  int32_t* viol = nullptr;
  hipError_t err = hipMalloc(&viol, (size_t)ngroups * sizeof(int32_t));
  if (err != hipSuccess) return (int)err;
  char* base = static_cast<char*>(e.blob);
  unsigned long long* acc = reinterpret_cast<unsigned long long*>(base + e.fp_offset);
  int rc = (int)queue_fingerprint(e.weight, weight_bytes(&e.desc, e.w_enc), acc, stream);
  if (rc == 0)
    rc = sengine_amd_compress_2_4(&e.desc, e.weight, e.w_enc, e.w_layout, base, base + e.value_bytes, viol, stream);
  std::vector<int32_t> host((size_t)ngroups);
  unsigned long long fp = 0;
  if (rc == 0) {
    err = hipMemcpyAsync(host.data(), viol, host.size() * sizeof(int32_t), hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipMemcpyAsync(&fp, acc, sizeof(fp), hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    rc = (int)err;
  }
  (void)hipFree(viol);
  if (rc) return rc;
  e.fingerprint = fp;
  e.valid = true;
  for (int32_t v : host)
    if (v) {
      e.valid = false;
      return sengine::set_error(-5, "prepare_weight: the weight is not 2:4 sparse along C_in (a 4-group holds "
                                    "more than two entries with |w| >= 1e-10)");
    }
  return 0;
}

// Fingerprint of the weight now (one synchronisation).
int current_fingerprint(const BlobEntry& e, hipStream_t stream, uint64_t* out) {
  unsigned long long* acc = reinterpret_cast<unsigned long long*>(static_cast<char*>(e.blob) + e.fp_offset);
  hipError_t err = queue_fingerprint(e.weight, weight_bytes(&e.desc, e.w_enc), acc, stream);
  unsigned long long fp = 0;
  if (err == hipSuccess) err = hipMemcpyAsync(&fp, acc, sizeof(fp), hipMemcpyDeviceToHost, stream);
  if (err == hipSuccess) err = hipStreamSynchronize(stream);
  *out = fp;
  return (int)err;
}

// The current blob of (device, weight, descriptor), built, checked or refreshed as described at
// the top of the file; *blob / *vb receive it.  Call with g_mu held.
int ensure_blob(const sengine_conv_lif_desc* d, const void* weight, int32_t w_enc, int32_t w_layout,
                hipStream_t stream, const char** blob, size_t* vb) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return (int)err;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  err = hipStreamIsCapturing(stream, &cs);
  if (err != hipSuccess) return (int)err;
  const bool capturing = cs != hipStreamCaptureStatusNone;
  BlobEntry* e = find_blob(dev, weight, d, w_enc, w_layout);
  if (e == nullptr) {
    if (capturing)
      return sengine::set_error(-4, "prepare_weight: the weight was not seen before stream capture began (call the "
                                    "node once outside capture, as the reference executor's warm-up does)");
    if (weight_bytes(d, w_enc) == 0 || weight_bytes(d, w_enc) % 4)
      return sengine::set_error(-2, "prepare_weight: weight encoding must be SENGINE_ENC_F16 or SENGINE_ENC_F32");
    size_t vbytes = 0, mbytes = 0;
    int rc = sengine_amd_sparse_blob_bytes(d, &vbytes, &mbytes);
    if (rc) return rc;
    BlobEntry ne{};
    ne.dev = dev;
    ne.weight = weight;
    ne.desc = *d;
    ne.w_enc = w_enc;
    ne.w_layout = w_layout;
    ne.value_bytes = vbytes;
    ne.fp_offset = (vbytes + mbytes + 255) / 256 * 256;
    if ((err = hipMalloc(&ne.blob, ne.fp_offset + 256)) != hipSuccess) return (int)err;
    rc = build_blob(ne, stream);
    if (rc) {
      (void)hipFree(ne.blob);
      return rc;
    }
    g_blobs.push_back(ne);
    e = &g_blobs.back();
  } else if (!capturing) {
    uint64_t fp = 0;
    int rc = current_fingerprint(*e, stream, &fp);
    if (rc) return rc;
    if (fp != e->fingerprint || !e->valid) {
      rc = build_blob(*e, stream);  // in place: graphs captured over this blob see the new weight
      if (rc) return rc;
    }
  } else if (!e->valid) {
    return sengine::set_error(-5, "fused_call_raw_weight: the weight's last eager check found it not 2:4 sparse "
                                  "along C_in");
  }
  *blob = static_cast<const char*>(e->blob);
  *vb = e->value_bytes;
  return 0;
}

}  // namespace

using namespace sengine;

extern "C" int sengine_amd_prepare_weight(const sengine_conv_lif_desc* d, const void* weight, int32_t w_enc,
                                          int32_t w_layout, hipStream_t stream) {
  if (!d || !weight) return set_error(-1, "prepare_weight: null descriptor or weight");
  std::lock_guard<std::mutex> lock(g_mu);
  const char* blob = nullptr;
  size_t vb = 0;
  return ensure_blob(d, weight, w_enc, w_layout, stream, &blob, &vb);
}

extern "C" int sengine_amd_fused_call_raw_weight(const sengine_conv_lif_desc* d, const void* data, const void* weight,
                                                 int32_t w_enc, int32_t w_layout, float* state, const float* bn_scale,
                                                 const float* bn_bias, void* spikes, hipStream_t stream) {
  if (!d || !weight) return set_error(-1, "fused_call_raw_weight: null descriptor or weight");
  const char* blob = nullptr;
  size_t vb = 0;
  {
    std::lock_guard<std::mutex> lock(g_mu);  // the table may grow meanwhile: copy the pointers out
    const int rc = ensure_blob(d, weight, w_enc, w_layout, stream, &blob, &vb);
    if (rc) return rc;
  }
  return sengine_amd_fused_sparse_conv_bn_lif(d, data, blob, blob + vb, state, bn_scale, bn_bias, spikes, nullptr,
                                              nullptr, stream);
}

extern "C" int sengine_amd_release_weights(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  int rc = 0;
  for (const BlobEntry& e : g_blobs) {
    int cur = 0;
    if (hipGetDevice(&cur) == hipSuccess && cur != e.dev) (void)hipSetDevice(e.dev);
    const hipError_t fe = hipFree(e.blob);
    if (fe != hipSuccess && rc == 0) rc = (int)fe;
    if (cur != e.dev) (void)hipSetDevice(cur);
  }
  g_blobs.clear();
  return rc;
}
