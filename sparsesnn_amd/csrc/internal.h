// Host-side helpers shared by the C-ABI entry points.
#pragma once
#include <stdint.h>

#include "common.h"

namespace sengine {

struct Geometry {
  int OH, OW;
  int64_t M;      // B*OH*OW rows per timestep
  int64_t K_red;  // KH*KW*C_in
};

// Records msg as this thread's last error and returns code (negative).
int set_error(int code, const char* msg);

// Validates a descriptor and derives the output geometry.  sparse=true adds the
// constraints of the 2:4 fused path (C_in % 64), otherwise the dense fallback's (C_in % 32).
int check_desc(const sengine_conv_lif_desc* d, Geometry* geo, bool sparse);

// Small-output ("flat") layout.  A convolution with at most kFlatMaxPixels output pixels
// per image, on an input not much larger than its kernel window, runs as one GEMM per image: rows = images (B per timestep), reduction over
// the whole input image in NHWC order (K_flat = H*W*C_in), columns = (output pixel,
// C_out) (N_flat = OH*OW*C_out), with the conv weights placed at the taps each output
// pixel sees and zeros elsewhere.  Input, output, membrane and trace memory are the
// ordinary NHWC tensors (same bytes).  The sparse blob of such a layer is built in this
// layout (sparse_blob_bytes / compress_2_4 use the same predicate), independent of the
// activation encoding.
constexpr int kFlatMaxPixels = 16;
constexpr int64_t kFlatMaxK = 16384;
constexpr int64_t kFlatMaxEntries = 1ll << 26;  // N_flat * K_flat
constexpr int64_t kFlatMaxWaste = 2;             // H*W <= 2*KH*KW (MACs vs the conv's)
constexpr int64_t kFlatMaxInflate = 4;           // OH*OW*H*W <= 4*KH*KW (weight entries vs the conv's)
bool flat_layout(const sengine_conv_lif_desc* d, const Geometry& geo);

// Paired-tail form of a 3x3 conv (the input's last 64-channel chunk holds 32 real channels):
// 0 if the descriptor takes it (3x3, stride 1, pad 1, no dilation, T = 4, spike bits in and
// out, one weight plane; checked after check_desc), else an error recorded under `who`.
int check_tail_desc(const sengine_conv_lif_desc* d, const char* who);
// Reduction chunks of its blob: 9 per full 64-channel chunk, then 5 tap pairs.
inline int tail_chunks(const sengine_conv_lif_desc* d) { return 9 * (d->C_in / 64 - 1) + 5; }

// Null if (neuron, tau) is a valid neuron description, else the reason.
const char* neuron_invalid(int neuron, float tau);

// fp32 neuron parameters with the rounding of the reference's python scalars:
// decay = float(1.0 - 1.0/tau) computed in double (models/neurons.py:124).
NeuronParams make_neuron_params(int neuron, int hard_reset, float tau, float vth, float vreset);

// Pointers of one fused call (already validated).
struct FusedArgs {
  const void* data;
  const void* wvals;
  const void* wmeta;
  float* state;
  const float* scale;
  const float* bias;
  void* out;
  float* h_trace;
  float* x_trace;
  SewAdd sew;  // fused SEW residual add (sew.res == nullptr: none)
};

// The paired-tail form on the persistent 3x3 kernel (fused_tile1.hip); describe_tail names
// its instance.
hipError_t launch_fused_bits_tail(const sengine_conv_lif_desc* d, const Geometry& geo, const FusedArgs& a, int mode,
                                  hipStream_t stream);
int describe_tail(const sengine_conv_lif_desc* d, const Geometry& geo, int mode, bool state, char* buf, size_t len);

// LDS-staged kernel for spike-bit inputs (fused_sparse_lds.hip).
hipError_t launch_fused_bits_lds(const sengine_conv_lif_desc* d, const Geometry& geo, const FusedArgs& a,
                                 hipStream_t stream);

// Tile kernels for spike-bit 3x3 / stride 1 / pad 1 and 1x1 / pad 0 convolutions with one
// weight plane and T <= 4 (tile_kernel.h, fused_tile1.hip, fused_tile3.hip).
bool tile_eligible(const sengine_conv_lif_desc* d);
hipError_t launch_fused_bits_tile(const sengine_conv_lif_desc* d, const Geometry& geo, const FusedArgs& a,
                                  hipStream_t stream);

// The tile kernel instance chosen for a descriptor (template arguments and grid).
struct TileChoice {
  bool k3;
  int shape, gpw, ksplit, pf;
  int tiles_w, tiles_per_image, ntiles;
  int pm;  // 1x1 only: channel groups per wave of the position-major kernel (0: the tile kernel)
  int pmw;  // position-major kernel: waves per workgroup (4 or 6)
  int cg;  // position-major kernel: 64-channel chunks per staging phase
};
bool choose_tile(const sengine_conv_lif_desc* d, const Geometry& geo, TileChoice& c);

// Direct-staged fp16-input 1x1 kernel (tile1ds.h, fused_tile1ds.hip): tile1ds_config returns its
// waves per workgroup (0: not eligible); the launch takes the tile route's TileParams.
struct TileParams;
int tile1ds_config(const sengine_conv_lif_desc* d, int64_t M, int mode, const FusedArgs* a);
int describe_tile1ds(const sengine_conv_lif_desc* d, int64_t M, int nw, int mode, bool state, char* buf,
                     size_t len);
hipError_t launch_fused_f16_tile1ds(const TileParams& p, const sengine_conv_lif_desc* d, int nw, int mode,
                                    hipStream_t stream);

// fp16 activations (T = 4, one weight plane) on geometries the tile forms do not cover: the
// gather form of the tile kernel (tile_kernel.h, KS = 0; fused_tile1.hip).
bool tile_gather_eligible(const sengine_conv_lif_desc* d);
hipError_t launch_fused_f16_gather(const sengine_conv_lif_desc* d, const Geometry& geo, const FusedArgs& a,
                                   hipStream_t stream);
int describe_gather(const sengine_conv_lif_desc* d, const Geometry& geo, int mode, char* buf, size_t len);

// Halo-tiled kernel for spike-bit 3x3 / stride 2 / pad 1 convolutions with one weight plane and
// T = 4 (tile3s.h, fused_tile3s.hip).
bool tile3s_eligible(const sengine_conv_lif_desc* d);
hipError_t launch_fused_bits_tile3s(const sengine_conv_lif_desc* d, const Geometry& geo, const FusedArgs& a,
                                    hipStream_t stream);
int describe_tile3s(const sengine_conv_lif_desc* d, const Geometry& geo, int mode, char* buf, size_t len);

// Human-readable names of the kernel instance a launch would run (snprintf semantics); `a`
// carries which optional buffers (state, traces, residuals) the launch passes.
int describe_tile(const sengine_conv_lif_desc* d, const Geometry& geo, int mode, bool shortcut_only,
                  const FusedArgs& a, char* buf, size_t len);
int describe_lds(const sengine_conv_lif_desc* d, const Geometry& geo, int mode, char* buf, size_t len);

// Kernel selection for the fused op with spike-bit input: 0 = automatic (the split-K
// small-M kernel for small outputs, else the tile kernel where eligible, else the
// LDS-staged kernel), 1 = always the direct-gather kernel, 2 = the LDS-staged kernel,
// 3 = the tile kernel where eligible (never small-M).  The flat small-output layout
// always takes the small-M kernel (direct for 1).  Read once from
// SENGINE_AMD_FUSED_KERNEL ("auto" | "direct" | "lds" | "tile").
int fused_kernel_choice();

}  // namespace sengine
