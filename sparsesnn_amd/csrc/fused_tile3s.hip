// Instantiations and host-side choice of the strided 3x3 halo-tiled kernel (tile3s.h).
#include "tile3s.h"

#include <stdio.h>
#include <stdlib.h>

namespace sengine {

namespace {

int env_now(const char* name, int dflt) {  // read per call: tests switch these between cases
  const char* e = getenv(name);
  return e ? atoi(e) : dflt;
}

struct Tile3sChoice {
  int shape;  // 0: 8x8 tiles, 1: 7x7
  int gpw, ksp;
  int tiles_w, tiles_per_image, ntiles;
};

constexpr int kShapeTR[2] = {8, 7};

// Relative cost of a tile shape for one image: SMFMAC issue over all position slots (valid or
// not) plus the halo staging (HBM words per chunk and timestep).
double s2_cost(int shape, int OH, int OW) {
  const int t = kShapeTR[shape];
  const int tiles = ((OH + t - 1) / t) * ((OW + t - 1) / t);
  const int halo = (2 * t + 1) * (2 * t + 1);
  return tiles * (64.0 * 9 * 4 * 26 / 16 + halo * 4 * 8.0);
}

bool choose(const sengine_conv_lif_desc* d, const Geometry& geo, Tile3sChoice& c) {
  const int fs = env_now("SENGINE_AMD_TILE3S_SHAPE", -1);
  c.shape = (fs == 0 || fs == 1) ? fs : (s2_cost(0, geo.OH, geo.OW) <= s2_cost(1, geo.OH, geo.OW) ? 0 : 1);
  const int t = kShapeTR[c.shape];
  c.tiles_w = (geo.OW + t - 1) / t;
  c.tiles_per_image = ((geo.OH + t - 1) / t) * c.tiles_w;
  c.ntiles = d->B * c.tiles_per_image;
  c.gpw = 1;  // one 64-channel group per wave (tile3s.h)
  // Reduction split over two wave sets for grids of at most one workgroup per CU (an even
  // number of 64-channel chunks).  SENGINE_AMD_TILE3S_KSP=1|2 overrides.
  const int nchunk = d->C_in / 64;
  c.ksp = (nchunk % 2 == 0 && (int64_t)c.ntiles * (d->C_out / (64 * c.gpw)) <= 256) ? 2 : 1;
  const int fk = env_now("SENGINE_AMD_TILE3S_KSP", 0);
  if (fk == 1 || (fk == 2 && nchunk % 2 == 0)) c.ksp = fk;
  return (int64_t)c.ntiles * (d->C_out / (64 * c.gpw)) <= 0x7fffffff;
}

template <int TR, int GPW>
hipError_t launch_ksp(const TileParams& p, int ksp, int out_enc, int mode, hipStream_t s) {
  return ksp == 2 ? launch_tile3s_shape<2, TR, TR, TR, GPW, 2>(p, out_enc, mode, s)
                  : launch_tile3s_shape<2, TR, TR, TR, GPW, 1>(p, out_enc, mode, s);
}

}  // namespace

// Spike-bit 3x3 / stride 2 / pad 1 convolutions with one weight plane and T = 4 (the first conv
// of a downsampling block).  SENGINE_AMD_TILE3S=0 turns the route off (the LDS-staged kernel
// then takes them).
bool tile3s_eligible(const sengine_conv_lif_desc* d) {
  if (env_now("SENGINE_AMD_TILE3S", 1) == 0) return false;
  if (d->in_enc != SENGINE_ENC_BITS || d->T != 4 || d->weight_planes != 1) return false;
  if (d->KH != 3 || d->KW != 3 || d->stride_h != 2 || d->stride_w != 2 || d->pad_h != 1 || d->pad_w != 1 ||
      d->dil_h != 1 || d->dil_w != 1)
    return false;
  // 32-bit input byte offsets in the kernel
  return (int64_t)d->T * d->B * d->H * d->W * (d->C_in / 8) < ((int64_t)1 << 31);
}

int describe_tile3s(const sengine_conv_lif_desc* d, const Geometry& geo, int mode, char* buf, size_t len) {
  Tile3sChoice c;
  if (!choose(d, geo, c)) return snprintf(buf, len, "none (grid too large)");
  static const char* const kEpi[] = {"generic", "lif_hard", "if_hard"};
  const bool bits = d->out_enc == SENGINE_ENC_BITS;
  const int t = kShapeTR[c.shape];
  return snprintf(buf, len, "tile3s<T=4,S=2,TR=%d,TC=%d,GPW=%d,KSP=%d,out=%s,epi=%s> grid=%lld", t, t, c.gpw, c.ksp,
                  bits ? "bits" : "f16", bits ? kEpi[mode] : "generic",
                  (long long)c.ntiles * (d->C_out / (64 * c.gpw)));
}

hipError_t launch_fused_bits_tile3s(const sengine_conv_lif_desc* d, const Geometry& geo, const FusedArgs& a,
                                    hipStream_t stream) {
  Tile3sChoice c;
  if (!choose(d, geo, c)) return hipErrorInvalidValue;
  TileParams p{};
  p.in = static_cast<const uint8_t*>(a.data);
  p.wvals = static_cast<const u32x4_t*>(a.wvals);
  p.wmeta = static_cast<const uint32_t*>(a.wmeta);
  p.state = a.state;
  p.scale = a.scale;
  p.bias = a.bias;
  p.out = static_cast<uint8_t*>(a.out);
  p.h_trace = a.h_trace;
  p.x_trace = a.x_trace;
  p.B = d->B; p.C = d->C_in; p.H = d->H; p.W = d->W; p.F = d->C_out;
  p.OH = geo.OH; p.OW = geo.OW; p.S = 2;
  p.M = (int)geo.M;
  p.nchunk = d->C_in / 64;
  p.nq = 9 * p.nchunk;
  p.np = make_neuron_params(d->neuron, d->hard_reset, d->tau, d->v_threshold, d->v_reset);
  p.enc_scale = 1.0f / kBitSpikeValue;
  p.sew = a.sew;
  p.tiles_w = c.tiles_w;
  p.tiles_per_image = c.tiles_per_image;
  p.ntiles = c.ntiles;
  const int mode = epilogue_mode(p.np, a.h_trace != nullptr || a.x_trace != nullptr || a.sew.real_out != nullptr);
  return c.shape == 0 ? launch_ksp<8, 1>(p, c.ksp, d->out_enc, mode, stream)
                      : launch_ksp<7, 1>(p, c.ksp, d->out_enc, mode, stream);
}

}  // namespace sengine
