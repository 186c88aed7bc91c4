// The reference runtime's weight tensor behind the fused call (host side).
//
// The reference's per-node call() receives the runtime's fp16 weight in (KH, KW, C_in, C_out)
// layout (sengine/cuda_graph_runtime.py:233-235, passed by sengine/csrc/cpp_executor.cu:
// 909-913).  This build's kernels read a 2:4 blob (SMFMAC-ordered values + metadata).  The
// entries below keep one blob per (device, weight pointer, descriptor): built on the first
// call outside stream capture (the reference executor runs every node eagerly three times
// before it captures, cpp_executor.cu:1270-1276), reused by every later call including the
// captured one.  A first call inside a capture is refused (it would have to allocate).
#include <mutex>
#include <vector>

#include "common.h"
#include "internal.h"

namespace {

struct BlobEntry {
  int dev;
  const void* weight;
  sengine_conv_lif_desc desc;
  int32_t w_enc, w_layout;
  void* blob;
  size_t value_bytes;
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

const BlobEntry* find_blob(int dev, const void* w, const sengine_conv_lif_desc* d, int32_t w_enc, int32_t w_layout) {
  for (const BlobEntry& e : g_blobs)
    if (e.dev == dev && e.weight == w && e.w_enc == w_enc && e.w_layout == w_layout && same_desc(e.desc, *d)) return &e;
  return nullptr;
}

}  // namespace

using namespace sengine;

extern "C" int sengine_amd_prepare_weight(const sengine_conv_lif_desc* d, const void* weight, int32_t w_enc,
                                          int32_t w_layout, hipStream_t stream) {
  if (!d || !weight) return set_error(-1, "prepare_weight: null descriptor or weight");
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  std::lock_guard<std::mutex> lock(g_mu);
  if (find_blob(dev, weight, d, w_enc, w_layout)) return 0;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(stream, &cs);
  if (e != hipSuccess) return (int)e;
  if (cs != hipStreamCaptureStatusNone)
    return set_error(-4, "prepare_weight: the weight was not seen before stream capture began (call the node once "
                         "outside capture, as the reference executor's warm-up does)");
  size_t vb = 0, mb = 0;
  int rc = sengine_amd_sparse_blob_bytes(d, &vb, &mb);
  if (rc) return rc;
  const int64_t ngroups = sengine_amd_num_groups(d);
  if (ngroups <= 0) return set_error(-2, "prepare_weight: invalid descriptor");
  void* blob = nullptr;
  int32_t* viol = nullptr;
  if ((e = hipMalloc(&blob, vb + mb)) != hipSuccess) return (int)e;
  if ((e = hipMalloc(&viol, (size_t)ngroups * sizeof(int32_t))) != hipSuccess) {
    (void)hipFree(blob);
    return (int)e;
  }
  rc = sengine_amd_compress_2_4(d, weight, w_enc, w_layout, blob, static_cast<char*>(blob) + vb, viol, stream);
  std::vector<int32_t> host((size_t)ngroups);
  if (rc == 0) {
    e = hipMemcpyAsync(host.data(), viol, host.size() * sizeof(int32_t), hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    rc = (int)e;
  }
  (void)hipFree(viol);
  if (rc == 0) {
    for (int32_t v : host)
      if (v) {
        rc = set_error(-5, "prepare_weight: the weight is not 2:4 sparse along C_in (a 4-group holds more than two "
                           "entries with |w| >= 1e-10)");
        break;
      }
  }
  if (rc) {
    (void)hipFree(blob);
    return rc;
  }
  g_blobs.push_back(BlobEntry{dev, weight, *d, w_enc, w_layout, blob, vb});
  return 0;
}

extern "C" int sengine_amd_fused_call_raw_weight(const sengine_conv_lif_desc* d, const void* data, const void* weight,
                                                 int32_t w_enc, int32_t w_layout, float* state, const float* bn_scale,
                                                 const float* bn_bias, void* spikes, hipStream_t stream) {
  if (!d || !weight) return set_error(-1, "fused_call_raw_weight: null descriptor or weight");
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  const char* blob = nullptr;
  size_t vb = 0;
  for (int pass = 0; pass < 2 && !blob; ++pass) {
    if (pass == 1) {
      const int rc = sengine_amd_prepare_weight(d, weight, w_enc, w_layout, stream);
      if (rc) return rc;
    }
    std::lock_guard<std::mutex> lock(g_mu);  // copy the entry out: the table may grow meanwhile
    if (const BlobEntry* be = find_blob(dev, weight, d, w_enc, w_layout)) {
      blob = static_cast<const char*>(be->blob);
      vb = be->value_bytes;
    }
  }
  if (!blob) return set_error(-1, "fused_call_raw_weight: weight blob missing after preparation");
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
