// Routing and launch of the direct-staged fp16 1x1 kernel (tile1ds.h).
#include <stdlib.h>

#include "tile1ds.h"

namespace sengine {
namespace {

int env_now(const char* name, int dflt) {  // read per call: tests switch these between cases
  const char* e = getenv(name);
  return e ? atoi(e) : dflt;
}

int cus_of_current_device() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  return n;
}

// Resident workgroups: two waves per SIMD -- two 4-wave workgroups per CU, or one 8-wave one.
int tile1ds_slots(int nw) {
  const int n = env_now("SENGINE_AMD_PS_SLOTS", 0);
  return n > 0 ? n : cus_of_current_device() * (nw == 8 ? 1 : 2);
}

template <int NW, int NCH>
hipError_t launch_nch(const TileParams& p, int oe, int mode, hipStream_t s) {
  if (oe == SENGINE_ENC_BITS) return launch_tile1ds<NW, NCH, SENGINE_ENC_BITS, false>(p, mode, tile1ds_slots(NW), s);
  return launch_tile1ds<NW, NCH, SENGINE_ENC_F16, true>(p, mode, tile1ds_slots(NW), s);
}

}  // namespace

// fp16-input 1x1 layers the kernel is written for: T = 4, stride 1, no padding, one weight
// plane, 16 | M, 4 or 6 input chunks, a fast hard-reset neuron, no trace or residual, 32-bit
// activation offsets; spike bits (optionally split into planes) or fp16 spikes out; a membrane
// state with fp16 output (the reference call's form, no split).  Waves per workgroup: 8 (512
// output channels share each staged activation) when 512 | C_out, else 4 when 256 | C_out.
// SENGINE_AMD_TILE1_DS=0 turns the route off.  Returns the waves per workgroup, or 0.
int tile1ds_config(const sengine_conv_lif_desc* d, int64_t M, int mode, const FusedArgs* a) {
  if (env_now("SENGINE_AMD_TILE1_DS", -1) == 0) return 0;
  const int nchunk = d->C_in / 64;
  if (d->in_enc != SENGINE_ENC_F16 || d->T != 4 || d->KH != 1 || d->KW != 1 || d->stride_h != 1 ||
      d->stride_w != 1 || d->pad_h != 0 || d->pad_w != 0 || d->weight_planes != 1 || d->C_in % 64 != 0 ||
      (nchunk != 4 && nchunk != 6) || M % 16 != 0 || (mode != EPI_LIF_HARD && mode != EPI_IF_HARD))
    return 0;
  if ((int64_t)d->T * M * d->C_in * 2 > 0x7fffffff) return 0;  // activation offsets are 32-bit
  if (a && (a->sew.res || a->sew.res16 || a->sew.real_out || a->h_trace || a->x_trace)) return 0;
  if (a && a->state && (d->out_enc != SENGINE_ENC_F16 || a->sew.split_c)) return 0;
  if (d->out_enc != SENGINE_ENC_BITS && d->out_enc != SENGINE_ENC_F16) return 0;
  if (d->C_out % 512 == 0) return 8;
  if (d->C_out % 256 == 0) return 4;
  return 0;
}

int describe_tile1ds(const sengine_conv_lif_desc* d, int64_t M, int nw, int mode, bool state, char* buf,
                     size_t len) {
  const int npg = (int)(M / 16), nsb = d->C_out / (64 * nw);
  const int per = tile1ps_per(npg, nsb, tile1ds_slots(nw));
  return snprintf(buf, len, "tile1ds<T=4,NW=%d,NCH=%d,in=f16,out=%s,epi=%s%s> grid=%d (persistent, %d groups)", nw,
                  d->C_in / 64, d->out_enc == SENGINE_ENC_BITS ? "bits" : "f16",
                  mode == EPI_LIF_HARD ? "lif_hard" : "if_hard", state ? ",state" : "", per * nsb, npg);
}

hipError_t launch_fused_f16_tile1ds(const TileParams& p, const sengine_conv_lif_desc* d, int nw, int mode,
                                    hipStream_t stream) {
  const int nch = d->C_in / 64;
  if (nw == 8) return nch == 4 ? launch_nch<8, 4>(p, d->out_enc, mode, stream)
                               : launch_nch<8, 6>(p, d->out_enc, mode, stream);
  return nch == 4 ? launch_nch<4, 4>(p, d->out_enc, mode, stream) : launch_nch<4, 6>(p, d->out_enc, mode, stream);
}

}  // namespace sengine
