// Host-side C-ABI utilities: versioning, error strings, geometry and blob sizes.
#include <math.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include "internal.h"

namespace sengine {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* msg) {
  snprintf(g_last_error, sizeof(g_last_error), "%s", msg);
  return code;
}

int check_desc(const sengine_conv_lif_desc* d, Geometry* geo, bool sparse) {
  if (!d) return set_error(-1, "null descriptor");
  if (d->T < 1 || d->B < 1 || d->C_in < 1 || d->H < 1 || d->W < 1 || d->C_out < 1)
    return set_error(-2, "T, B, C_in, H, W, C_out must be >= 1");
  if (d->KH < 1 || d->KW < 1 || d->stride_h < 1 || d->stride_w < 1 || d->dil_h < 1 || d->dil_w < 1 ||
      d->pad_h < 0 || d->pad_w < 0)
    return set_error(-2, "kernel/stride/dilation must be >= 1 and padding >= 0");
  const int OH = (d->H + 2 * d->pad_h - d->dil_h * (d->KH - 1) - 1) / d->stride_h + 1;
  const int OW = (d->W + 2 * d->pad_w - d->dil_w * (d->KW - 1) - 1) / d->stride_w + 1;
  if (OH < 1 || OW < 1) return set_error(-2, "empty output spatial extent");
  if (sparse && d->C_in % 64 != 0) return set_error(-2, "sparse path requires C_in % 64 == 0");
  if (!sparse && d->C_in % 32 != 0) return set_error(-2, "dense path requires C_in % 32 == 0");
  if (d->C_out % 64 != 0) return set_error(-2, "C_out % 64 == 0 required");
  if (d->weight_planes != 1 && d->weight_planes != 2) return set_error(-2, "weight_planes must be 1 or 2");
  if (const char* why = neuron_invalid(d->neuron, d->tau)) return set_error(-2, why);
  const int64_t pixels = (int64_t)d->T * d->B * d->H * d->W;
  if (pixels * d->C_in > (1ll << 40)) return set_error(-2, "input too large");
  geo->OH = OH;
  geo->OW = OW;
  geo->M = (int64_t)d->B * OH * OW;
  geo->K_red = (int64_t)d->KH * d->KW * d->C_in;
  return 0;
}

int check_tail_desc(const sengine_conv_lif_desc* d, const char* who) {
  static thread_local char msg[192];
  const char* why = nullptr;
  if (d->KH != 3 || d->KW != 3 || d->stride_h != 1 || d->stride_w != 1 || d->pad_h != 1 || d->pad_w != 1 ||
      d->dil_h != 1 || d->dil_w != 1)
    why = "needs a 3x3 kernel, stride 1, padding 1, no dilation";
  else if (d->T != 4)
    why = "needs T = 4";
  else if (d->in_enc != SENGINE_ENC_BITS || d->out_enc != SENGINE_ENC_BITS)
    why = "needs spike bits in and out";
  else if (d->weight_planes != 1)
    why = "needs one weight plane";
  else if ((int64_t)d->T * d->B * d->H * d->W * (d->C_in / 8) >= ((int64_t)1 << 31))
    why = "input too large for 32-bit offsets";
  if (!why) return 0;
  snprintf(msg, sizeof msg, "%s: %s", who, why);
  return set_error(-2, msg);
}

bool flat_layout(const sengine_conv_lif_desc* d, const Geometry& geo) {
  const int64_t npix = (int64_t)geo.OH * geo.OW;
  const int64_t kf = (int64_t)d->H * d->W * d->C_in;
  const int64_t nf = npix * d->C_out;
  // the flat matrix multiplies H*W / (KH*KW) times the conv's own work (taps outside the
  // window are zeros): allowed up to kFlatMaxWaste
  const bool cheap = (int64_t)d->H * d->W <= kFlatMaxWaste * d->KH * d->KW;
  // ... and holds OH*OW*H*W / (KH*KW) times the conv's weight entries, all read every call
  const bool compact = npix * d->H * d->W <= kFlatMaxInflate * d->KH * d->KW;
  return npix <= kFlatMaxPixels && kf <= kFlatMaxK && nf * kf <= kFlatMaxEntries && cheap && compact;
}

static int g_kernel_choice = -1;

int fused_kernel_choice() {
  if (g_kernel_choice < 0) {
    const char* e = getenv("SENGINE_AMD_FUSED_KERNEL");
    g_kernel_choice = !e                         ? 0
                      : strcmp(e, "direct") == 0 ? 1
                      : strcmp(e, "lds") == 0    ? 2
                      : strcmp(e, "tile") == 0   ? 3
                                                 : 0;
  }
  return g_kernel_choice;
}

const char* neuron_invalid(int neuron, float tau) {
  if (neuron != SENGINE_NEURON_LIF && neuron != SENGINE_NEURON_IF && neuron != SENGINE_NEURON_MS)
    return "neuron must be LIF, IF or MS";
  if (neuron == SENGINE_NEURON_LIF && !(tau > 0.f)) return "LIF tau must be > 0";
  if (neuron == SENGINE_NEURON_MS && !(tau >= 0.f && tau <= 1.f)) return "MS decay (tau field) must be in [0, 1]";
  return nullptr;
}

NeuronParams make_neuron_params(int neuron, int hard_reset, float tau, float vth, float vreset) {
  if (neuron == SENGINE_NEURON_MS) {
    // h = v*decay + x is the LIF recurrence with x/tau = x (tau 1) and the given decay:
    // fma(v, decay, x) when v*decay is exact (decay a power of two or zero), else the
    // separately rounded product and sum, like torch's mem * decay + x.
    NeuronParams np;
    np.neuron = SENGINE_NEURON_LIF;
    np.hard_reset = hard_reset;
    np.tau = 1.0f;
    np.vth = vth;
    np.vreset = vreset;
    np.decay = tau;
    np.rtau = 1.0f;
    int e;
    const double dm = frexp((double)tau, &e);
    np.pow2 = (tau == 0.0f || dm == 0.5) ? 1 : 0;
    return np;
  }
  NeuronParams np;
  np.neuron = neuron;
  np.hard_reset = hard_reset;
  np.tau = tau;
  np.vth = vth;
  np.vreset = vreset;
  np.pow2 = 0;
  np.rtau = 1.0f;
  np.decay = 1.0f;
  if (neuron == SENGINE_NEURON_LIF) {
    const double t = (double)tau;
    np.decay = (float)(1.0 - 1.0 / t);
    int e;
    const double mant = frexp(1.0 / t, &e);
    // 1/tau exactly a power of two and the decay product exact (|decay| a power of two
    // or zero): then x/tau == x*rtau and v*decay needs no rounding.
    const bool rt_pow2 = mant == 0.5;
    int e2;
    const double dm = frexp((double)np.decay, &e2);
    const bool decay_pow2 = np.decay == 0.0f || dm == 0.5 || dm == -0.5;
    if (rt_pow2 && decay_pow2 && (double)np.decay == 1.0 - 1.0 / t) {
      np.pow2 = 1;
      np.rtau = (float)(1.0 / t);
    }
  }
  return np;
}

}  // namespace sengine

using namespace sengine;

extern "C" int sengine_amd_version(void) { return 100; }

extern "C" const char* sengine_amd_last_error(void) { return g_last_error; }

extern "C" int sengine_amd_set_fused_kernel(int32_t choice) {
  if (choice < 0 || choice > 3)
    return set_error(-2, "set_fused_kernel: choice must be 0 (auto), 1 (direct), 2 (lds) or 3 (tile)");
  g_kernel_choice = choice;
  return 0;
}

extern "C" int sengine_amd_conv_geometry(const sengine_conv_lif_desc* d, int32_t* OH, int32_t* OW,
                                         int64_t* M_per_t, int64_t* K_red) {
  if (!d) return set_error(-1, "null descriptor");
  Geometry geo;
  // geometry only: validate the shape fields, not the channel-divisibility rules
  if (d->T < 1 || d->B < 1 || d->C_in < 1 || d->H < 1 || d->W < 1 || d->C_out < 1 || d->KH < 1 ||
      d->KW < 1 || d->stride_h < 1 || d->stride_w < 1 || d->dil_h < 1 || d->dil_w < 1 || d->pad_h < 0 ||
      d->pad_w < 0)
    return set_error(-2, "invalid shape fields");
  geo.OH = (d->H + 2 * d->pad_h - d->dil_h * (d->KH - 1) - 1) / d->stride_h + 1;
  geo.OW = (d->W + 2 * d->pad_w - d->dil_w * (d->KW - 1) - 1) / d->stride_w + 1;
  if (geo.OH < 1 || geo.OW < 1) return set_error(-2, "empty output spatial extent");
  if (OH) *OH = geo.OH;
  if (OW) *OW = geo.OW;
  if (M_per_t) *M_per_t = (int64_t)d->B * geo.OH * geo.OW;
  if (K_red) *K_red = (int64_t)d->KH * d->KW * d->C_in;
  return 0;
}

extern "C" int sengine_amd_sparse_blob_bytes(const sengine_conv_lif_desc* d, size_t* value_bytes,
                                             size_t* meta_bytes) {
  Geometry geo;
  int rc = check_desc(d, &geo, true);
  if (rc) return rc;
  const bool flat = flat_layout(d, geo);
  const size_t groups = (size_t)(flat ? (int64_t)geo.OH * geo.OW * d->C_out : d->C_out) / 64;
  const size_t nq = (size_t)((flat ? (int64_t)d->H * d->W * d->C_in : geo.K_red) / 64);
  // per (group, chunk, plane, tile): 64 lanes x 8 fp16; per (group, chunk, tile): 64 lanes x u32
  if (value_bytes) *value_bytes = groups * nq * d->weight_planes * 4 * 64 * 16;
  if (meta_bytes) *meta_bytes = groups * nq * 4 * 64 * 4;
  return 0;
}

extern "C" int sengine_amd_tail_blob_bytes(const sengine_conv_lif_desc* d, size_t* value_bytes, size_t* meta_bytes) {
  Geometry geo;
  int rc = check_desc(d, &geo, true);
  if (rc) return rc;
  if ((rc = check_tail_desc(d, "tail_blob_bytes"))) return rc;
  const size_t groups = (size_t)d->C_out / 64, nq = (size_t)tail_chunks(d);
  if (value_bytes) *value_bytes = groups * nq * 4 * 64 * 16;
  if (meta_bytes) *meta_bytes = groups * nq * 4 * 64 * 4;
  return 0;
}

extern "C" int sengine_amd_dense_blob_bytes(const sengine_conv_lif_desc* d, size_t* value_bytes) {
  Geometry geo;
  int rc = check_desc(d, &geo, false);
  if (rc) return rc;
  const size_t groups = (size_t)d->C_out / 64;
  const size_t nq = (size_t)(geo.K_red / 32);
  if (value_bytes) *value_bytes = groups * nq * d->weight_planes * 4 * 64 * 16;
  return 0;
}

extern "C" int64_t sengine_amd_num_groups(const sengine_conv_lif_desc* d) {
  if (!d || d->C_in % 4 != 0) return -1;
  return (int64_t)d->C_out * d->KH * d->KW * (d->C_in / 4);
}
