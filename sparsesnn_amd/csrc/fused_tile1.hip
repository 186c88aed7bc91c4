// Instantiations of the tile kernel (tile_kernel.h) for 1x1 / pad 0 convolutions (any
// stride), and the host-side choice between tile shapes and channel blocking.
#include "tile1pm.h"
#include "tile1ps.h"
#include "tile_kernel.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

namespace sengine {

hipError_t launch_tile1(const TileParams& p, int T, int gpw, int oe, int mode, hipStream_t s) {
  switch (T) {
    case 1:
      return launch_tile<1, 1, 0, 0, 1, 1>(p, oe, mode, s);
    case 2:
      return launch_tile<2, 1, 0, 0, 1, 1>(p, oe, mode, s);
    case 4:
      return gpw == 2 ? launch_tile<4, 1, 0, 0, 1, 2>(p, oe, mode, s) : launch_tile<4, 1, 0, 0, 1, 1>(p, oe, mode, s);
    default:
      return hipErrorInvalidValue;
  }
}

namespace {

constexpr TileShape kShapes3[] = {{3, 8, 8, 8}, {3, 14, 4, 8}, {3, 7, 7, 7}};

int env_int_now(const char* name, int dflt) {  // read per call: tests switch these between cases
  const char* e = getenv(name);
  return e ? atoi(e) : dflt;
}

// Relative cost of a 3x3 tile shape: SMFMAC issue over all position slots (valid or not)
// plus the halo expansion (~72 VALU ops of ~4 cycles per 64-bit spike word), per image.
double shape_cost(const TileShape& s, int H, int W) {
  const int tiles = ((H + s.TR - 1) / s.TR) * ((W + s.TC - 1) / s.TC);
  const int slots = 16 * ((s.TC + 1) / 2) * ((s.TR + s.GR - 1) / s.GR);
  const double mfma = (double)slots / 16 * 9 * 4 * 26;
  const double stage = (double)(s.TR + 2) * (s.TC + 2) * 4 * 72.0 / 64 * 4;
  return tiles * (mfma + stage);
}

}  // namespace

bool tile_eligible(const sengine_conv_lif_desc* d) {
  if (d->weight_planes != 1 || d->dil_h != 1 || d->dil_w != 1) return false;
  if (d->in_enc != SENGINE_ENC_BITS && !(d->in_enc == SENGINE_ENC_F16 && d->T == 4)) return false;
  // fp16 input: 32-bit byte offsets of the fp16 rows
  if (d->in_enc == SENGINE_ENC_F16 && (int64_t)d->T * d->B * d->H * d->W * d->C_in * 2 >= ((int64_t)1 << 31))
    return false;
  // 32-bit input offsets in the kernel
  if ((int64_t)d->T * d->B * d->H * d->W * (d->C_in / 8) >= ((int64_t)1 << 31)) return false;
  if (d->T != 1 && d->T != 2 && d->T != 4) return false;
  const bool k3 = d->KH == 3 && d->KW == 3 && d->stride_h == 1 && d->stride_w == 1 && d->pad_h == 1 && d->pad_w == 1;
  const bool k1 = d->KH == 1 && d->KW == 1 && d->pad_h == 0 && d->pad_w == 0 && d->stride_h == d->stride_w;
  return k3 || k1;
}

// The tile kernel instance for a descriptor: tile shape, channel groups per wave, reduction
// split and prefetch depth (the launchers' template arguments) and the grid.  False when
// the grid would not fit.
bool choose_tile(const sengine_conv_lif_desc* d, const Geometry& geo, TileChoice& c) {
  c.k3 = d->KH == 3;
  c.shape = 0;
  if (c.k3) {
    if (d->T == 4) {
      const int forced = env_int_now("SENGINE_AMD_TILE_SHAPE", -1);  // tuning: 0, 1, 2
      if (forced >= 0 && forced < 3) {
        c.shape = forced;
      } else {
        double best = 0;
        for (int i = 0; i < 3; ++i) {
          const double cost = shape_cost(kShapes3[i], geo.OH, geo.OW);
          if (i == 0 || cost < best) best = cost, c.shape = i;
        }
      }
    }
    const TileShape s = kShapes3[c.shape];
    c.tiles_w = (geo.OW + s.TC - 1) / s.TC;
    c.tiles_per_image = ((geo.OH + s.TR - 1) / s.TR) * c.tiles_w;
    c.ntiles = d->B * c.tiles_per_image;
  } else {
    c.tiles_w = c.tiles_per_image = 0;
    c.ntiles = (int)((geo.M + 63) / 64);
  }

  // Two 64-channel groups per wave halve the B bytes per SMFMAC but double the
  // accumulators (2 waves per SIMD instead of 3) and halve the workgroup count; used when
  // the grid still gives every CU two workgroups.  SENGINE_AMD_TILE_GPW=1|2 overrides.
  c.gpw = (!c.k3 && d->T == 4 && d->C_out % 128 == 0 && (int64_t)c.ntiles * (d->C_out / 128) >= 512) ? 2 : 1;
  const int fg = env_int_now("SENGINE_AMD_TILE_GPW", 0);
  if (d->T == 4 && d->C_out % 128 == 0 && (fg == 1 || fg == 2)) c.gpw = fg;
  if ((int64_t)c.ntiles * (d->C_out / (64 * c.gpw)) > 0x7fffffff) return false;

  // Split the reduction over two wave sets when the grid gives at most one workgroup per
  // CU (deep layers: few, long workgroups, one wave per SIMD); with more workgroups the
  // doubled LDS footprint costs more than it gains (measured).  SENGINE_AMD_TILE_KSPLIT
  // =1|2 overrides.
  c.ksplit = 1;
  if (c.k3 && d->T == 4 && c.gpw == 1 && (d->C_in / 64) % 2 == 0) {
    c.ksplit = (int64_t)c.ntiles * (d->C_out / 64) <= 256 ? 2 : 1;
    const int fk = env_int_now("SENGINE_AMD_TILE_KSPLIT", 0);
    if (fk == 1 || fk == 2) c.ksplit = fk;
  }
  // Two-deep operand prefetch where the grid leaves at most two workgroups per CU (two waves
  // per SIMD: registers to spare, SMFMAC issue waiting on latency).  SENGINE_AMD_TILE_PF=1|2
  // overrides.
  c.pf = 1;
  if (c.k3 && d->T == 4 && c.gpw == 1) {
    c.pf = (int64_t)c.ntiles * (d->C_out / 64) <= 512 ? 2 : 1;
    const int fp = env_int_now("SENGINE_AMD_TILE_PF", 0);
    if (fp == 1 || fp == 2) c.pf = fp;
  }
  // 1x1, T = 4: the position-major kernel (tile1pm.h) when the channels split into 4 waves of
  // 128 (or 64) channels and the reduction into phases of 4 (or 2) chunks.
  // SENGINE_AMD_TILE1_PM=0|1|2 forces the tile kernel, or that many channel groups per wave.
  c.pm = 0;
  c.pmw = 4;
  c.cg = 0;
  const int nchunk = d->C_in / 64;
  c.cg = nchunk % 4 == 0 ? 4 : (nchunk % 2 == 0 ? 2 : 0);
  if (d->in_enc == SENGINE_ENC_F16) {  // fp16 input: one channel group per wave, one-tap prefetch
    c.gpw = 1;
    if (!c.k3) c.ksplit = 1;  // 3x3: the reduction split above (even chunk count, small grids)
    c.pf = 1;
    // 1x1: the position-major kernel stages each fp16 value once per 384 or 256 output
    // channels (6 or 4 waves), phases of 2 chunks (4 chunks hold too many prefetch registers)
    c.cg = 0;
    if (!c.k3 && d->T == 4 && nchunk % 2 == 0 && env_int_now("SENGINE_AMD_TILE1_PM", -1) != 0) {
      c.pmw = d->C_out % 384 == 0 ? 6 : (d->C_out % 256 == 0 ? 4 : 0);
      if (c.pmw && ((geo.M + 15) / 16) * (int64_t)(d->C_out / (64 * c.pmw)) <= 0x7fffffff) {
        c.pm = 1;
        c.cg = 2;
      }
    }
    return true;
  }
  if (!c.k3 && d->T == 4 && c.cg > 0) {
    c.pm = d->C_out % 512 == 0 ? 2 : (d->C_out % 256 == 0 ? 1 : 0);
    const int fpm = env_int_now("SENGINE_AMD_TILE1_PM", -1);
    if (fpm == 0 || (fpm == 1 && d->C_out % 256 == 0) || (fpm == 2 && d->C_out % 512 == 0)) c.pm = fpm;
    if (c.pm && ((geo.M + 15) / 16) * (int64_t)(d->C_out / (256 * c.pm)) > 0x7fffffff) c.pm = 0;
  }
  return true;
}

// The membrane-shortcut launches (fp32 y stored, no traces, bit output, no SEW residual) of the
// 3x3 T = 4 tile kernel with one channel group per wave take the lean EPI_SHORTCUT epilogue.
static int tile_epilogue_mode(const sengine_conv_lif_desc* d, const TileChoice& c, int mode, bool shortcut_only) {
  if (shortcut_only && c.k3 && d->T == 4 && c.gpw == 1 && d->in_enc == SENGINE_ENC_BITS &&
      d->out_enc == SENGINE_ENC_BITS)
    return EPI_SHORTCUT;
  return mode;
}

// Compute units of the current device (cached per device; the persistent 1x1 kernel sizes its
// grid to the resident workgroups).
static int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// The persistent 1x1 kernel (tile1ps.h) serves the token Linears when a layer is what it is
// written for: stride 1, T = 4, 16 | M, an even chunk count, a fast hard-reset neuron, no trace
// or bit-plane residual.  fp16 input with spike-bit or fp16 output (q/k/v and fc1; the
// exported per-node call's fp16-in, fp16-out 1x1 layers), no fp16 residual: 256-channel
// super-blocks (4 waves, phases of 2 chunks) or 384-channel ones (6 waves, phases of 3 chunks,
// an even phase count).  Spike-bit input with fp16 output, optionally + the fp16 residual (proj,
// fc2) or spike bits (1x1 layers of convolutional networks): 384-channel super-blocks with
// phases of 6 chunks, or 256-channel ones with 4.  A membrane state (the reference executor's
// call) is served on the fp16-in, fp16-out and the bits-in, bits-out forms.  Stateless spike-bit
// input on 384-channel super-blocks with 32 | M takes 32-position groups (phases of 3 chunks:
// each A operand feeds twice the SMFMACs); SENGINE_AMD_TILE1_NPG=1 keeps 16-position groups.
// SENGINE_AMD_TILE1_PS=0 turns it off.  Returns 256 * (position groups per group - 1) + waves *
// 16 + chunks per phase, or 0.
static int tile1ps_config(const sengine_conv_lif_desc* d, const Geometry& geo, const TileChoice& c, int mode,
                          const FusedArgs* a) {
  const int nchunk = d->C_in / 64;
  const int env = env_int_now("SENGINE_AMD_TILE1_PS", -1);
  if (env == 0 || c.k3 || d->T != 4 || d->stride_h != 1 || d->stride_w != 1 || d->weight_planes != 1 ||
      geo.M % 16 != 0 || nchunk % 2 != 0 || (mode != EPI_LIF_HARD && mode != EPI_IF_HARD))
    return 0;
  if (a && (a->sew.res || a->sew.real_out || a->h_trace || a->x_trace)) return 0;
  if (a && a->state && (d->in_enc != d->out_enc || a->sew.res16 || a->sew.split_c)) return 0;
  if (d->in_enc == SENGINE_ENC_F16) {
    if (!c.pm || (a && a->sew.res16)) return 0;
    if ((int64_t)d->T * geo.M * d->C_in * 2 > 0x7fffffff) return 0;  // piece offsets are 32-bit
    if (d->C_out % 256 == 0) return 4 * 16 + 2;
    if (d->C_out % 384 == 0 && nchunk % 6 == 0) return 6 * 16 + 3;
    return 0;
  }
  if (d->in_enc != SENGINE_ENC_BITS) return 0;
  if (d->out_enc == SENGINE_ENC_BITS && a && a->sew.res16) return 0;
  if (d->C_out % 384 == 0 && nchunk % 6 == 0) {
    if (geo.M % 32 == 0 && !(a && a->state) && env_int_now("SENGINE_AMD_TILE1_NPG", 2) == 2) return 256 + 6 * 16 + 3;
    return 6 * 16 + 6;
  }
  if (d->C_out % 256 == 0 && nchunk % 4 == 0) return 4 * 16 + 4;
  return 0;
}

// Resident workgroups of the persistent kernel (two waves per SIMD): two 4-wave workgroups per
// CU, or one 6-wave workgroup (the waves of a second would not all find a SIMD).
static int tile1ps_slots(int nw) {
  const int n = env_int_now("SENGINE_AMD_PS_SLOTS", 0);
  return n > 0 ? n : device_cus() * (nw == 6 ? 1 : 2);
}

// The persistent 3x3 kernel (tile3ps.h) takes the tile launches it is written for: T = 4, spike
// bits in and out, one channel group per wave, no reduction split, one-tap prefetch, a fast
// hard-reset neuron (with or without a membrane state), no trace or residual, and at least two
// tiles per resident workgroup (three per CU).  SENGINE_AMD_TILE3_PS=0 turns it off, =2 lifts the two-tile rule.
// SENGINE_AMD_PS_SLOTS=n launches the persistent kernels on n workgroups instead (tests use it
// to make small layers walk several tiles or groups per workgroup).
static int ps_slots_override() { return env_int_now("SENGINE_AMD_PS_SLOTS", 0); }
static int tile3ps_slots() { return ps_slots_override() > 0 ? ps_slots_override() : device_cus() * 3; }
static bool tile3ps_eligible(const sengine_conv_lif_desc* d, const TileChoice& c, int mode, const FusedArgs* a) {
  if (!c.k3 || d->T != 4 || d->in_enc != SENGINE_ENC_BITS || d->out_enc != SENGINE_ENC_BITS || c.gpw != 1 ||
      c.ksplit != 1 || c.pf != 1 || (mode != EPI_LIF_HARD && mode != EPI_IF_HARD))
    return false;
  // at least two tiles per resident workgroup: with fewer, the hardware's dispatch of a partial
  // second round of one-tile workgroups balances the CUs better than a fixed assignment
  // (measured); and one input chunk: with two or three the halo-tiled kernel measured faster
  // (Spikformer's 128 -> 192 224^2 and 192 -> 384 112^2 convs, 1,192 against 1,243 us and 842
  // against 890).  SENGINE_AMD_TILE3_PS=2 waives both rules.
  const int env = env_int_now("SENGINE_AMD_TILE3_PS", -1);
  if (env == 0) return false;
  if (env != 2 && ((int64_t)c.ntiles * (d->C_out / 64) < 2LL * tile3ps_slots() || d->C_in != 64)) return false;
  // (its epilogue stores plain spike-bit rows: no SEW sum, no channel-split planes)
  if (a && (a->sew.res || a->sew.res16 || a->sew.real_out || a->sew.split_c || a->h_trace || a->x_trace))
    return false;
  return true;
}

int describe_tile(const sengine_conv_lif_desc* d, const Geometry& geo, int mode, bool shortcut_only,
                  const FusedArgs& a, char* buf, size_t len) {
  TileChoice c;
  if (!choose_tile(d, geo, c)) return snprintf(buf, len, "none (grid too large)");
  mode = tile_epilogue_mode(d, c, mode, shortcut_only);
  static const char* const kEpi[] = {"generic", "lif_hard", "if_hard", "shortcut"};
  const char* oe = d->out_enc == SENGINE_ENC_BITS ? "bits" : "f16";
  const bool f16in = d->in_enc == SENGINE_ENC_F16;
  // fp16 output runs the generic epilogue except in launch_tile's 1x1 fast case and the fp16-input
  // tile instances (every mode)
  const bool fast_f16out = f16in ? c.pm == 0 : (d->T == 4 && c.pm == 0 && mode == EPI_LIF_HARD);
  const char* epi = d->out_enc == SENGINE_ENC_BITS || fast_f16out ? kEpi[mode] : "generic";
  if (!c.k3)
    if (const int nw = tile1ds_config(d, geo.M, mode, &a))
      return describe_tile1ds(d, geo.M, nw, mode, a.state != nullptr, buf, len);
  if (const int ps = tile1ps_config(d, geo, c, mode, &a)) {
    const int nw = (ps >> 4) & 15, gp = 16 * (1 + (ps >> 8)), npg = (int)(geo.M / gp), nsb = d->C_out / (64 * nw);
    const int per = tile1ps_per(npg, nsb, tile1ps_slots(nw));
    return snprintf(buf, len, "tile1ps<T=4,NW=%d,CG=%d,in=%s,out=%s,epi=%s%s%s> grid=%d (persistent, %d groups)", nw,
                    ps & 15, f16in ? "f16" : "bits", oe, kEpi[mode], a.state ? ",state" : "", gp == 32 ? ",pos=32" : "",
                    per * nsb, npg);
  }
  if (f16in && c.pm)
    return snprintf(buf, len, "tile1pm<T=4,GPW=1,CG=2,NW=%d,in=f16,out=%s,epi=%s> grid=%lld", c.pmw, oe, epi,
                    (long long)((geo.M + 15) / 16) * (d->C_out / (64 * c.pmw)));
  if (f16in) {
    if (c.k3) {
      const TileShape s = kShapes3[c.shape];
      return snprintf(buf, len, "tile<T=4,KS=3,TR=%d,TC=%d,GR=%d,GPW=1,KSP=%d,PF=1,in=f16,out=%s,epi=%s> grid=%lld",
                      s.TR, s.TC, s.GR, c.ksplit, oe, epi, (long long)c.ntiles * (d->C_out / 64));
    }
    return snprintf(buf, len, "tile<T=4,KS=1,GPW=1,in=f16,out=%s,epi=%s> grid=%lld", oe, epi,
                    (long long)c.ntiles * (d->C_out / 64));
  }
  if (c.k3 && tile3ps_eligible(d, c, mode, &a)) {
    const TileShape s = kShapes3[c.shape];
    const int ncb = d->C_out / 64;
    const int per = std::max(1, std::min(tile3ps_slots() / ncb, c.ntiles));
    return snprintf(buf, len, "tile3ps<T=4,TR=%d,TC=%d,GR=%d,out=bits,epi=%s%s> grid=%d (persistent, %d tiles)",
                    s.TR, s.TC, s.GR, kEpi[mode], a.state ? ",state" : "", per * ncb, c.ntiles);
  }
  if (c.k3) {
    const TileShape s = kShapes3[c.shape];
    return snprintf(buf, len, "tile<T=%d,KS=3,TR=%d,TC=%d,GR=%d,GPW=%d,KSP=%d,PF=%d,out=%s,epi=%s> grid=%lld",
                    d->T, s.TR, s.TC, s.GR, c.gpw, c.ksplit, c.pf, oe, epi,
                    (long long)c.ntiles * (d->C_out / (64 * c.gpw)));
  }
  if (c.pm)
    return snprintf(buf, len, "tile1pm<T=%d,GPW=%d,CG=%d,out=%s,epi=%s> grid=%lld", d->T, c.pm, c.cg, oe, epi,
                    (long long)((geo.M + 15) / 16) * (d->C_out / (256 * c.pm)));
  return snprintf(buf, len, "tile<T=%d,KS=1,GPW=%d,out=%s,epi=%s> grid=%lld", d->T, c.gpw, oe, epi,
                  (long long)c.ntiles * (d->C_out / (64 * c.gpw)));
}

bool tile_gather_eligible(const sengine_conv_lif_desc* d) {
  if (d->in_enc != SENGINE_ENC_F16 || d->T != 4 || d->weight_planes != 1 || tile_eligible(d)) return false;
  if (env_int_now("SENGINE_AMD_GATHER", 1) == 0) return false;  // =0: the direct-gather kernel instead
  // 32-bit byte offsets of the fp16 rows; 16-bit receptive-field origins
  return (int64_t)d->T * d->B * d->H * d->W * d->C_in * 2 < ((int64_t)1 << 31) && d->H < 16384 && d->W < 16384;
}

int describe_gather(const sengine_conv_lif_desc* d, const Geometry& geo, int mode, char* buf, size_t len) {
  static const char* const kEpi[] = {"generic", "lif_hard", "if_hard"};
  return snprintf(buf, len, "tile<T=4,KS=0(gather %dx%d/%d),GPW=1,in=f16,out=%s,epi=%s> grid=%lld", d->KH, d->KW,
                  d->stride_h, d->out_enc == SENGINE_ENC_BITS ? "bits" : "f16", kEpi[mode],
                  (long long)((geo.M + 63) / 64) * (d->C_out / 64));
}

hipError_t launch_fused_f16_gather(const sengine_conv_lif_desc* d, const Geometry& geo, const FusedArgs& a,
                                   hipStream_t stream) {
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
  p.OH = geo.OH; p.OW = geo.OW; p.S = d->stride_h;
  p.KW = d->KW; p.SH = d->stride_h; p.SW = d->stride_w; p.PH = d->pad_h; p.PW = d->pad_w;
  p.DH = d->dil_h; p.DW = d->dil_w;
  p.M = (int)geo.M;
  p.nchunk = d->C_in / 64;
  p.nq = d->KH * d->KW * p.nchunk;
  p.np = make_neuron_params(d->neuron, d->hard_reset, d->tau, d->v_threshold, d->v_reset);
  p.enc_scale = 1.0f;
  p.sew = a.sew;
  p.ntiles = (int)((geo.M + 63) / 64);
  const int mode = epilogue_mode(p.np, a.h_trace != nullptr || a.x_trace != nullptr || a.sew.real_out != nullptr);
  return launch_tile_f16in<0, 0, 0, 1>(p, d->out_enc, mode, stream);
}

static TileParams tile_params(const sengine_conv_lif_desc* d, const Geometry& geo, const FusedArgs& a,
                              const TileChoice& c) {
  TileParams p;
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
  p.OH = geo.OH; p.OW = geo.OW; p.S = d->stride_h;
  p.M = (int)geo.M;
  p.nchunk = d->C_in / 64;
  p.nq = d->KH * d->KW * p.nchunk;
  p.np = make_neuron_params(d->neuron, d->hard_reset, d->tau, d->v_threshold, d->v_reset);
  p.enc_scale = d->in_enc == SENGINE_ENC_BITS ? 1.0f / kBitSpikeValue : 1.0f;
  p.sew = a.sew;
  p.tiles_w = c.tiles_w;
  p.tiles_per_image = c.tiles_per_image;
  p.ntiles = c.ntiles;
  return p;
}

hipError_t launch_fused_bits_tail(const sengine_conv_lif_desc* d, const Geometry& geo, const FusedArgs& a, int mode,
                                  hipStream_t stream) {
  TileChoice c;
  if (!choose_tile(d, geo, c) || !c.k3) return hipErrorInvalidValue;
  TileParams p = tile_params(d, geo, a, c);
  p.nq = tail_chunks(d);
  return launch_tile3_persistent_pair(p, c.shape, mode, tile3ps_slots(), stream);
}

int describe_tail(const sengine_conv_lif_desc* d, const Geometry& geo, int mode, bool state, char* buf, size_t len) {
  TileChoice c;
  if (!choose_tile(d, geo, c) || !c.k3) return snprintf(buf, len, "none (grid too large)");
  static const char* const kEpi[] = {"generic", "lif_hard", "if_hard"};
  const TileShape s = kShapes3[c.shape];
  const int ncb = d->C_out / 64;
  const int per = std::max(1, std::min(tile3ps_slots() / ncb, c.ntiles));
  return snprintf(buf, len, "tile3ps<T=4,TR=%d,TC=%d,GR=%d,out=bits,epi=%s%s,pair> grid=%d (persistent, %d tiles, "
                  "%d reduction chunks)", s.TR, s.TC, s.GR, kEpi[mode], state ? ",state" : "", per * ncb, c.ntiles,
                  tail_chunks(d));
}

hipError_t launch_fused_bits_tile(const sengine_conv_lif_desc* d, const Geometry& geo, const FusedArgs& a,
                                  hipStream_t stream) {
  TileChoice c;
  if (!choose_tile(d, geo, c)) return hipErrorInvalidValue;
  TileParams p = tile_params(d, geo, a, c);
  const bool shortcut_only = a.sew.real_out != nullptr && a.h_trace == nullptr && a.x_trace == nullptr &&
                             a.sew.res == nullptr;
  const int mode = tile_epilogue_mode(
      d, c, epilogue_mode(p.np, a.h_trace != nullptr || a.x_trace != nullptr || a.sew.real_out != nullptr),
      shortcut_only);
  if (d->in_enc == SENGINE_ENC_F16) {
    if (c.k3) return launch_tile3_f16in(p, c.shape, c.ksplit, d->out_enc, mode, stream);
    if (const int nw = tile1ds_config(d, geo.M, mode, &a)) return launch_fused_f16_tile1ds(p, d, nw, mode, stream);
    if (const int ps = tile1ps_config(d, geo, c, mode, &a)) {
      if (d->out_enc == SENGINE_ENC_F16)  // fp16 in and out: the exported per-node call's form (with state)
        return ps == 6 * 16 + 3
                   ? launch_tile1ps<6, 3, SENGINE_ENC_F16, SENGINE_ENC_F16, 0, true>(p, mode, tile1ps_slots(6), stream)
                   : launch_tile1ps<4, 2, SENGINE_ENC_F16, SENGINE_ENC_F16, 0, true>(p, mode, tile1ps_slots(4), stream);
      return ps == 6 * 16 + 3 ? launch_tile1ps<6, 3, SENGINE_ENC_F16, SENGINE_ENC_BITS>(p, mode, tile1ps_slots(6), stream)
                              : launch_tile1ps<4, 2, SENGINE_ENC_F16, SENGINE_ENC_BITS>(p, mode, tile1ps_slots(4), stream);
    }
    if (c.pm)
      return c.pmw == 6 ? launch_tile1pm<4, 1, 2, 6, SENGINE_ENC_F16>(p, d->out_enc, mode, stream)
                        : launch_tile1pm<4, 1, 2, 4, SENGINE_ENC_F16>(p, d->out_enc, mode, stream);
    return launch_tile_f16in<1, 0, 0, 1>(p, d->out_enc, mode, stream);
  }
  if (c.k3 && tile3ps_eligible(d, c, mode, &a)) return launch_tile3_persistent(p, c.shape, mode, tile3ps_slots(), stream);
  if (c.k3) return launch_tile3(p, d->T, c.shape, c.gpw, c.ksplit, c.pf, d->out_enc, mode, stream);
  if (const int ps = tile1ps_config(d, geo, c, mode, &a)) {
    const int nw = (ps >> 4) & 15;
    if (ps >> 8)  // 32-position groups, 384-channel super-blocks
      return d->out_enc == SENGINE_ENC_F16
                 ? launch_tile1ps<6, 3, SENGINE_ENC_BITS, SENGINE_ENC_F16, 0, false, 2>(p, mode, tile1ps_slots(6), stream)
                 : launch_tile1ps<6, 3, SENGINE_ENC_BITS, SENGINE_ENC_BITS, 0, false, 2>(p, mode, tile1ps_slots(6), stream);
    if (d->out_enc == SENGINE_ENC_F16)
      return nw == 6 ? launch_tile1ps<6, 6, SENGINE_ENC_BITS, SENGINE_ENC_F16>(p, mode, tile1ps_slots(6), stream)
                     : launch_tile1ps<4, 4, SENGINE_ENC_BITS, SENGINE_ENC_F16>(p, mode, tile1ps_slots(4), stream);
    if (nw == 6)
      return launch_tile1ps<6, 6, SENGINE_ENC_BITS, SENGINE_ENC_BITS, 0, true>(p, mode, tile1ps_slots(6), stream);
    // one 4-chunk phase (C_in = 256): the A operands stay resident
    return p.nchunk == 4
               ? launch_tile1ps<4, 4, SENGINE_ENC_BITS, SENGINE_ENC_BITS, 1, true>(p, mode, tile1ps_slots(4), stream)
               : launch_tile1ps<4, 4, SENGINE_ENC_BITS, SENGINE_ENC_BITS, 0, true>(p, mode, tile1ps_slots(4), stream);
  }
  if (c.pm == 2) return c.cg == 4 ? launch_tile1pm<4, 2, 4>(p, d->out_enc, mode, stream)
                                  : launch_tile1pm<4, 2, 2>(p, d->out_enc, mode, stream);
  if (c.pm == 1) return c.cg == 4 ? launch_tile1pm<4, 1, 4>(p, d->out_enc, mode, stream)
                                  : launch_tile1pm<4, 1, 2>(p, d->out_enc, mode, stream);
  return launch_tile1(p, d->T, c.gpw, d->out_enc, mode, stream);
}

}  // namespace sengine
