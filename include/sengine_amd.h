/*
 * sengine_amd.h — C ABI of the MI355X (gfx950) fused 2:4-sparse Conv+BN+LIF operator.
 *
 * Every entry point takes plain device pointers, plain integers and a HIP stream,
 * never allocates device memory, never synchronises, and returns 0 on success.
 * A negative return is an argument error detected on the host (nothing was
 * launched; sengine_amd_last_error() describes it); a positive return is the
 * hipError_t reported by the launch.  All launches are safe under stream capture.
 *
 * Reference interfaces replaced (paths relative to the SparseSNN repository):
 *   - the per-node kernel ABI `int init(void)` / `int call(ptrs..., stream)`
 *     exported by sengine/build/export_standalone.py:1-8,37-103 and dlopen'd by
 *     sengine/csrc/cpp_executor.cu:631-662, called with six pointers
 *     (data, weight, state, bn_scale, bn_bias, spikes) at cpp_executor.cu:909-913;
 *   - the fused operator conv2d_bn_if_interleaved_kernel
 *     (sengine/kernels/conv2d_bn_if_t4.py:918-1022) and conv1x1_bn_lif / conv1x1_bn_if
 *     (sengine/kernels/interleaved_templates.py:28-154), i.e. the node variants
 *     KernelVariant.FusedSparseConvBNLIF / TileLangFusedConvBNIF /
 *     TileLangFusedConv1x1BNIF (sengine/ir.py:53,78-79);
 *   - the unfused fallback conv2d_bn_t4_kernel / conv1x1_bn_t4_kernel
 *     (sengine/kernels/conv2d_bn_if_t4.py:551-673) followed by lif_neuron_kernel /
 *     if_neuron_kernel (sengine/csrc/kernels.cuh:18-54).
 *
 * Data layouts (all NHWC, rows ordered t-major then b, oh, ow — the order of
 * models/layers.py:26-31 SeqToANNContainer and of the reference kernels):
 *   spike bits : uint32 words, position p = ((t*B + b)*H + h)*W + w holds C/32 words;
 *                channel c is bit (c % 32) of word c/32.
 *   fp16 dense : _Float16 [(t*B + b)*H + h][w][c]  (the reference's io dtype).
 *   membrane   : float [B*OH*OW][C_out]  (cuda_graph_runtime.py:385-390).
 *   BN         : folded per-channel scale / bias, fp32 (sengine/optimizer.py:159-183).
 *   weights    : an opaque "sparse blob" produced by sengine_amd_compress_2_4
 *                (2:4 values in SMFMAC operand order + 2-bit position metadata),
 *                or a "dense blob" from sengine_amd_pack_dense_weights.
 */
#ifndef SENGINE_AMD_H
#define SENGINE_AMD_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Activation / spike encodings. */
enum {
  SENGINE_ENC_BITS = 0, /* 1 bit per value, value = bit (binary spikes) */
  SENGINE_ENC_F16 = 1,  /* fp16 NHWC (any fp16 value on input; 0.0 / 1.0 on output) */
  SENGINE_ENC_F32 = 2   /* fp32 NHWC (pack/unpack and weights only) */
};

/* Neuron models (sengine/ir.py:44-48 NeuronType, models/neurons.py). */
/* LIF: h = v*(1 - 1/tau) + x/tau (models/neurons.py:121-146); IF: h = v + x;
 * MS: h = v*decay + x with decay carried in the descriptor's `tau` field -- the MS-ResNet
 * neuron mem = mem*decay*(1 - spike) + x (models/msresnet.py:28-56) with hard_reset = 1,
 * v_reset = 0.  All fire when h >= v_threshold. */
enum { SENGINE_NEURON_LIF = 0, SENGINE_NEURON_IF = 1, SENGINE_NEURON_MS = 2 };

/* Weight tensor layouts accepted by the compressors. */
enum {
  SENGINE_WLAYOUT_OIHW = 0, /* torch nn.Conv2d weight (C_out, C_in, KH, KW) */
  SENGINE_WLAYOUT_HWIO = 1  /* reference runtime layout (KH, KW, C_in, C_out), cuda_graph_runtime.py:233-235 */
};

/*
 * Shape + neuron descriptor of one Conv+BN+LIF node.  Mirrors ConvParams +
 * NeuronParams (sengine/ir.py:179-201) plus the batch/time extents the
 * reference bakes into each compiled kernel (tilelang_compiler.py:551-553).
 */
typedef struct sengine_conv_lif_desc {
  int32_t T, B;                 /* timesteps, batch */
  int32_t C_in, H, W, C_out;    /* input channels/spatial, output channels */
  int32_t KH, KW;               /* kernel */
  int32_t stride_h, stride_w;
  int32_t pad_h, pad_w;
  int32_t dil_h, dil_w;
  int32_t neuron;               /* SENGINE_NEURON_LIF / _IF / _MS */
  int32_t hard_reset;           /* 1: v <- v_reset after a spike; 0: v <- v - v_threshold */
  float tau, v_threshold, v_reset; /* tau: LIF time constant; MS: the decay factor */
  int32_t in_enc;               /* SENGINE_ENC_BITS or SENGINE_ENC_F16 */
  int32_t out_enc;              /* SENGINE_ENC_BITS or SENGINE_ENC_F16 */
  int32_t weight_planes;        /* 1: fp16 weights; 2: fp16 hi + fp16 lo (fp32-faithful) */
} sengine_conv_lif_desc;

/* Library version (major*10000 + minor*100 + patch). */
int sengine_amd_version(void);

/* Human-readable description of the last negative return on this thread. */
const char* sengine_amd_last_error(void);

/*
 * Kernel selection for sengine_amd_fused_sparse_conv_bn_lif with spike-bit input:
 * 0 = automatic (the default: a split-K small-M kernel when the output has fewer than 128
 * units of 64 positions x 64 channels, else the tile kernel for 3x3 / stride 1 / pad 1 and
 * 1x1 / pad 0 with one weight plane and T <= 4, else the LDS-staged kernel), 1 =
 * direct-gather kernel (the kernel fp16 inputs always use), 2 = LDS-staged kernel, 3 =
 * tile kernel where eligible (never small-M).  Convs in the flat small-output layout (at
 * most 16 output pixels, an input at most 2x the kernel window and a flat matrix of at most
 * 4x the conv's weight entries) use its kernels for every choice.  Process-wide; the
 * environment variable SENGINE_AMD_FUSED_KERNEL=direct|lds|tile sets 1|2|3 at load time.
 * Every choice computes the same operator (the tests hold each one to the same oracle).
 */
int sengine_amd_set_fused_kernel(int32_t choice);

/* Output spatial size, M = B*OH*OW rows per timestep and K_red = KH*KW*C_in. */
int sengine_amd_conv_geometry(const sengine_conv_lif_desc* d, int32_t* OH, int32_t* OW,
                              int64_t* M_per_t, int64_t* K_red);

/*
 * Byte sizes of the weight blobs for a descriptor (sparse: values + metadata;
 * dense: values).  The fused kernel reads the sparse blob; the fallback the dense one.
 */
int sengine_amd_sparse_blob_bytes(const sengine_conv_lif_desc* d, size_t* value_bytes, size_t* meta_bytes);
int sengine_amd_dense_blob_bytes(const sengine_conv_lif_desc* d, size_t* value_bytes);

/*
 * 2:4 weight compressor (new in this build; the reference only validates 2:4,
 * sengine/optimizer.py:499-553, and leaves compression to TensorRT).
 * weight: fp32 (w_enc = SENGINE_ENC_F32) or fp16 (SENGINE_ENC_F16) in layout w_layout.
 * Each group of 4 consecutive input channels at one (c_out, kh, kw) must hold at most
 * two entries with |w| >= 1e-10 (the zero test of validate_2_4_pattern); entries below
 * that are dropped.  violations (device, optional): receives, per 4-group, 1 if the
 * group had more than two such entries (the group is then truncated to its first two).
 * The blob is laid out for the descriptor's C_out/C_in/KH/KW and weight_planes only.
 */
int sengine_amd_compress_2_4(const sengine_conv_lif_desc* d, const void* weight, int32_t w_enc,
                             int32_t w_layout, void* blob_values, void* blob_meta,
                             int32_t* violations, hipStream_t stream);

/* Number of 4-groups the compressor checks (= C_out*KH*KW*C_in/4): size of `violations`. */
int64_t sengine_amd_num_groups(const sengine_conv_lif_desc* d);

/* Dense weight packer for the unfused fallback (any weights). */
int sengine_amd_pack_dense_weights(const sengine_conv_lif_desc* d, const void* weight, int32_t w_enc,
                                   int32_t w_layout, void* blob_values, hipStream_t stream);

/*
 * Fused 2:4-sparse Conv + folded BN + multi-step LIF/IF over T (one launch).
 * Replaces conv2d_bn_if_interleaved_kernel / conv1x1_bn_lif (see above).
 *   data     : input activations, encoding d->in_enc, (T*B, H, W, C_in)
 *   blob_*   : from sengine_amd_compress_2_4
 *   state    : optional (may be NULL => V0 = 0, not written back) fp32 (B*OH*OW, C_out);
 *              read as the initial membrane and overwritten with the final one.
 *   bn_scale, bn_bias : fp32 (C_out)
 *   spikes   : output, encoding d->out_enc, (T*B, OH, OW, C_out)
 *   h_trace  : optional fp32 (T, B*OH*OW, C_out): charged membrane at each t (pre-reset)
 *   x_trace  : optional fp32 (T, B*OH*OW, C_out): BN output (LIF input current)
 * Requires C_in % 64 == 0, C_out % 64 == 0, T in {1,2,4,8}.
 */
/*
 * The fused call with its spike bits split by channel into planes of split_channels:
 * output channel c goes to plane c / split_channels, channel c % split_channels, each plane a
 * (T*B*OH*OW, split_channels) bit matrix, planes back to back (ceil(C_out / split_channels)
 * of them).  For several layers that read the same input and were concatenated along C_out
 * (Spikformer's q, k and v Linears, models/spikformer.py:72-86): one launch, each layer's
 * spikes in its own tensor.  split_channels % 64 == 0; spike-bit output; no traces; not in
 * the flat small-output layout.  Same values as sengine_amd_fused_sparse_conv_bn_lif.
 */
int sengine_amd_fused_sparse_conv_bn_lif_split(const sengine_conv_lif_desc* d, const void* data,
                                               const void* blob_values, const void* blob_meta, float* state,
                                               const float* bn_scale, const float* bn_bias, void* spikes,
                                               int32_t split_channels, hipStream_t stream);

int sengine_amd_fused_sparse_conv_bn_lif(const sengine_conv_lif_desc* d, const void* data,
                                         const void* blob_values, const void* blob_meta,
                                         float* state, const float* bn_scale, const float* bn_bias,
                                         void* spikes, float* h_trace, float* x_trace,
                                         hipStream_t stream);

/*
 * Names the kernel instance that sengine_amd_fused_sparse_conv_bn_lif (and its _add /
 * _add_neuron forms) would launch for descriptor d, without launching anything: the
 * route (tile / lds / smallm / direct) and its compile-time specialisation, e.g.
 * "tile<T=4,KS=3,TR=7,TC=7,GR=7,GPW=1,KSP=2,PF=2,out=bits,epi=lif_hard> grid=256".
 * flags: SENGINE_PLAN_* bits saying which optional buffers the call would pass (traces,
 * state, a SEW residual, the membrane-shortcut output).  Honours the same environment
 * switches and sengine_amd_set_fused_kernel choice as a launch.  Host-only (no GPU
 * needed).  This build's own introspection: the reference's compiler records the chosen
 * TileLang config on the node instead (sengine/build/tilelang_compiler.py:537,649).
 * Returns 0, or a negative code when d is invalid or buf (len bytes) is too small.
 */
#define SENGINE_PLAN_TRACES 1
#define SENGINE_PLAN_STATE 2
#define SENGINE_PLAN_SEW_ADD 4
#define SENGINE_PLAN_SHORTCUT 8
#define SENGINE_PLAN_TAIL 16 /* the paired-tail call, sengine_amd_fused_sparse_conv_bn_lif_tail */
int sengine_amd_fused_plan(const sengine_conv_lif_desc* d, int32_t flags, char* buf, size_t len);

/*
 * Paired-tail form of the fused 3x3 call, for a conv whose input channels were padded up to a
 * multiple of 64 by 32 zero channels (Spikformer's SPS proj_conv2 reads embed/4 = 96 channels,
 * models/spikformer.py:159-165; the same operator as conv2d_bn_if_interleaved_kernel,
 * sengine/kernels/conv2d_bn_if_t4.py:918-1022).  The descriptor is the padded conv (C_in a
 * multiple of 64); its input's channels C_in - 32 .. C_in - 1 are never read, and their weights
 * must be zero.  Each 64-deep reduction step of the last chunk takes the 32 real channels of
 * two taps, so that chunk costs 5 steps instead of 9 (9 * (C_in / 64 - 1) + 5 in all).
 * 3x3, stride 1, pad 1, no dilation, T = 4, spike bits in and out, one weight plane, a
 * hard-reset IF or LIF (power-of-two tau); no traces.  state as in the fused call.
 *   tail_blob_bytes : blob sizes of this form (fewer chunks than sparse_blob_bytes)
 *   compress_2_4_tail: its 2:4 compressor (arguments as compress_2_4; violations also flags
 *                      every group of four of the last 32 channels holding a weight with
 *                      |w| >= 1e-10)
 *   fused_sparse_conv_bn_lif_tail: the call; same values as the fused call on the padded
 *                      conv and blob up to the order of the fp32 sums (within the parity
 *                      tolerance, not bit for bit)
 */
int sengine_amd_tail_blob_bytes(const sengine_conv_lif_desc* d, size_t* value_bytes, size_t* meta_bytes);
int sengine_amd_compress_2_4_tail(const sengine_conv_lif_desc* d, const void* weight, int32_t w_enc,
                                  int32_t w_layout, void* blob_values, void* blob_meta, int32_t* violations,
                                  hipStream_t stream);
int sengine_amd_fused_sparse_conv_bn_lif_tail(const sengine_conv_lif_desc* d, const void* data,
                                              const void* blob_values, const void* blob_meta, float* state,
                                              const float* bn_scale, const float* bn_bias, void* spikes,
                                              hipStream_t stream);

/*
 * Two fused Conv + BN + neuron nodes that read the same input `data` -- a residual block's
 * conv1 and its 1x1 downsample (models/sewresnet.py:50-66: conv1 -> bn1 -> sn1 and
 * downsample(x) on the same x) -- with the results of sengine_amd_fused_sparse_conv_bn_lif
 * (d0, data, values0, meta0, NULL, scale0, bias0, spikes0, NULL, NULL) followed by the same
 * for d1 (bit-identical).  Both descriptors must share T, B, C_in, H, W and in_enc.  When both
 * convs run on the split-K small-output kernel with the same epilogue, it is one launch (a
 * launch each otherwise).  No state or traces.
 */
int sengine_amd_fused_sparse_conv_bn_lif_pair(const sengine_conv_lif_desc* d0, const sengine_conv_lif_desc* d1,
                                              const void* data, const void* values0, const void* meta0,
                                              const float* bn_scale0, const float* bn_bias0, void* spikes0,
                                              const void* values1, const void* meta1, const float* bn_scale1,
                                              const float* bn_bias1, void* spikes1, hipStream_t stream);

/*
 * Fused Conv + BN + neuron with the SEW 'ADD' residual connection in the epilogue:
 * out = spike + residual (models/sewresnet.py:58-59; replaces conv2d_bn_if_add_t4_kernel,
 * sengine/kernels/conv2d_bn_if_t4.py:813-911, whose output is fp16 spike + residual).
 * Integer-valued activations are stored as bit planes interleaved per position: a tensor
 * with P planes is an NHWC spike-bit tensor with P*C channels, channel p*C + c holding bit p
 * of channel c's value.  residual: (T*B, OH, OW) positions x residual_planes*C_out bits;
 * out: out_planes*C_out bits per position; 1 <= residual_planes <= out_planes <= 5 and the
 * caller chooses out_planes so that spike + residual fits (SEW-ResNet-18: up to 3 planes;
 * Spikformer's residual stream: up to 5).
 * A conv whose input is such a P-plane tensor is an ordinary spike-bit conv with C_in =
 * P*C and weights [W, 2W, 4W, ...] along the input channels (sparsesnn_amd.sparsity).
 * out_enc = F16 is the reference kernel's own form: out is fp16 NHWC (T*B, OH, OW, C_out),
 * out = spike + residual (exact for integer values below 2048), the residual fp16 of the same
 * shape when residual_planes == 0, else residual_planes bit planes as above; out_planes is
 * ignored; C_out % 32 == 0.  state may be NULL; no traces.
 */
int sengine_amd_fused_sparse_conv_bn_lif_add(const sengine_conv_lif_desc* d, const void* data,
                                             const void* blob_values, const void* blob_meta, float* state,
                                             const float* bn_scale, const float* bn_bias, const void* residual,
                                             int32_t residual_planes, void* out, int32_t out_planes,
                                             hipStream_t stream);

/*
 * Membrane-shortcut epilogue (MS-ResNet, models/msresnet.py:107-112,164-167; the reference
 * engine's Add+LIF fusion, sengine/kernels/add_lif_fused.py): y = BN(conv(data)) +
 * residual, stored as fp32 NHWC real_out (T*B, OH, OW, C_out) -- the block output that
 * carries the shortcut stream -- and the neuron of d run over y (V0 = state or 0), its
 * spikes stored in `spikes` (d->out_enc).  residual: fp32 (T*B, OH, OW, C_out), or NULL
 * for y = BN(conv).  No traces; any kernel / geometry of sengine_amd_fused_sparse_conv_bn_lif.
 */
int sengine_amd_fused_sparse_conv_bn_add_neuron(const sengine_conv_lif_desc* d, const void* data,
                                                const void* blob_values, const void* blob_meta, float* state,
                                                const float* bn_scale, const float* bn_bias, const float* residual,
                                                float* real_out, void* spikes, hipStream_t stream);

/*
 * Real-valued shortcut of an MS-ResNet block (BasicBlock18.shortcut: TDBNContainer(Conv2d
 * 1x1 / stride s, BatchNorm3d), models/msresnet.py:113-118, applied at :111 to the block's
 * real-valued input, not to spikes): out = conv1x1(x) * bn_scale + bn_bias in fp32.
 * x: fp32 NHWC (in_T*B, H, W, C_in); out: fp32 NHWC (T*B, OH, OW, C_out).  in_T = 1 takes
 * one timestep of input (the stem output, which the reference repeats over T before the
 * first block, :146-150) and stores each output value T times; in_T = d->T maps timestep
 * to timestep.  weight: OIHW (C_out, C_in, 1, 1) or HWIO (1, 1, C_in, C_out) fp32 (dense:
 * a 2:4-pruned weight runs with its zeros).  Needs KH = KW = 1, pad 0, equal strides,
 * C_in % 16 == 0, C_out % 64 == 0.
 */
int sengine_amd_real_conv_bn(const sengine_conv_lif_desc* d, const float* x, int32_t in_T, const float* weight,
                             int32_t w_layout, const float* bn_scale, const float* bn_bias, float* out,
                             hipStream_t stream);

/*
 * Spiking self-attention (Spikformer SSA, models/spikformer.py:103-130): for every (t, b,
 * head) x = (Q K^T * scale) V on binary spikes, then the neuron over T (the reference's
 * attn_lif: LIF tau 2, V_th 0.5).  Every product and partial sum is an integer times
 * `scale` (a power of two), exact in fp32 in any order; this library evaluates
 * Q (K^T V) * scale, which is bit-identical and costs N*d^2 instead of N^2*d per head.
 * q/k/v/out: spike bits (T*B, N, C), head h = channels [h*d, h*d + d), d = C/heads
 * (d % 16 == 0, d <= 64, N <= 8192, T in {1, 2, 4, 8}; a workgroup of the attend step keeps
 * K^T V of every t, 288*T*d bytes, and the Q slices of its token range, 8*T bytes per token --
 * ranges of at least 64 tokens, about 1024*N/(B*heads) when B*heads < 1024 -- in LDS, together
 * at most 160 KB, else -2).  Two steps:
 *   sengine_amd_ssa_kv:             kv (T*B, heads, d, d) int32 = K^T V   (caller's workspace)
 *   sengine_amd_ssa_attend_neuron:  out = neuron over T of (Q kv * scale)
 */
int sengine_amd_ssa_kv(int32_t T, int32_t B, int32_t N, int32_t C, int32_t heads, const uint32_t* k_bits,
                       const uint32_t* v_bits, int32_t* kv, hipStream_t stream);
int sengine_amd_ssa_attend_neuron(int32_t T, int32_t B, int32_t N, int32_t C, int32_t heads, float scale,
                                  int32_t neuron, int32_t hard_reset, float tau, float v_threshold, float v_reset,
                                  const uint32_t* q_bits, const int32_t* kv, uint32_t* out_bits, hipStream_t stream);

/*
 * Allocation-free spiking self-attention: sengine_amd_ssa_kv followed by
 * sengine_amd_ssa_attend_neuron with the K^T V partial sums in a library-owned device array
 * instead of a caller workspace.  No counterpart in the reference: for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * The array holds at most 4,194,304 int32 (16 MiB, T * B * heads * (C/heads)^2 entries; larger
 * calls return -2), every GPU the library runs on keeps one until the process ends, and the
 * call allocates nothing (the array's address is looked up once per device).  All calls on
 * one GPU share the array: calls that overlap on that GPU (other streams, or threads) race.
 * Arguments and results as the two entries above.
 */
int sengine_amd_ssa_attention_noalloc(int32_t T, int32_t B, int32_t N, int32_t C, int32_t heads, float scale,
                                      int32_t neuron, int32_t hard_reset, float tau, float v_threshold, float v_reset,
                                      const uint32_t* q_bits, const uint32_t* k_bits, const uint32_t* v_bits,
                                      uint32_t* out_bits, hipStream_t stream);

/*
 * Dense stem convolution on images + folded BN (the reference runs it through cuDNN,
 * sengine/csrc/cpp_executor.cu:306-347; models/sewresnet.py:140-141,199-200):
 * x NCHW fp32 (d->B images, d->C_in, d->H, d->W), weight fp32 in w_layout (HWIO reads
 * coalesced, OIHW does not), out NHWC fp32 (d->B, OH, OW, d->C_out).  Any C_in / kernel /
 * stride / pad (dilation 1); T is ignored.
 */
int sengine_amd_stem_conv_bn(const sengine_conv_lif_desc* d, const float* x, const float* weight, int32_t w_layout,
                             const float* bn_scale, const float* bn_bias, float* out, hipStream_t stream);

/*
 * The stem, its neuron and the max-pool in one launch (models/sewresnet.py:199-203: conv1,
 * bn1, repeat over T, sn1, maxpool): conv + folded BN as sengine_amd_stem_conv_bn (HWIO
 * weights), the neuron of d (V0 = 0) on that output repeated over d->T, then
 * MaxPool2d(pool_k, pool_stride, pool_pad) of the spikes.  pooled: (T, B, POH, POW) x
 * C_out bits; spikes (optional, may be NULL): the stem spikes (T, B, OH, OW) x C_out bits.
 * Bit-identical to the three separate entry points.  Needs C_out % 32 == 0, T <= 16,
 * OH*OW <= 256 and the image's staged input rows within LDS (a 3x32x32 image with a 7x7/2
 * stem fits); returns -2 otherwise.
 */
int sengine_amd_stem_conv_bn_lif_pool(const sengine_conv_lif_desc* d, const float* x, const float* weight,
                                      const float* bn_scale, const float* bn_bias, int32_t pool_k,
                                      int32_t pool_stride, int32_t pool_pad, uint32_t* spikes, uint32_t* pooled,
                                      hipStream_t stream);

/*
 * The stem and the neuron over its output repeated T times in one launch (MS-ResNet:
 * models/msresnet.py:135-138 conv1, :146-150 the image repeated over T, :119-120 the first
 * block's sn1 on that output and its shortcut on the same real-valued output): conv +
 * folded BN as sengine_amd_stem_conv_bn (HWIO weights) into out (optional, may be NULL: NHWC
 * fp32 (B, OH, OW, C_out)), and the neuron of d (V0 = 0) on it repeated over d->T into
 * spikes (T, B, OH, OW) x C_out bits, the layout of sengine_amd_multistep_neuron_repeat on
 * that out.  3-channel 7x7 or 3x3 stems of 32 or 64 channels run on the fp32 matrix cores:
 * out then agrees with sengine_amd_stem_conv_bn to fp32 summation order, and the spikes are
 * bit-identical to sengine_amd_multistep_neuron_repeat on this out; other stems (or the
 * environment switch SENGINE_AMD_STEM_MFMA=0) are bit-identical to those two entry points
 * with sengine_amd_stem_conv_bn's own out.  Needs C_out % 32 == 0 and the input
 * rows of 256 consecutive output pixels within LDS (3 channels of 224-wide images with a
 * 7x7/2 or 3x3/1 stem fit); returns -2 otherwise.
 */
int sengine_amd_stem_conv_bn_neuron(const sengine_conv_lif_desc* d, const float* x, const float* weight,
                                    const float* bn_scale, const float* bn_bias, float* out, uint32_t* spikes,
                                    hipStream_t stream);

/*
 * Multi-step neuron on an input repeated at every timestep (the stem output,
 * x.unsqueeze(0).repeat(T), models/sewresnet.py:201-202): x fp32 (n), V0 = 0,
 * spikes bits (T, n); n % 32 == 0.
 */
int sengine_amd_multistep_neuron_repeat(int32_t T, int64_t n, int32_t neuron, int32_t hard_reset, float tau,
                                        float v_threshold, float v_reset, const float* x, uint32_t* spikes,
                                        hipStream_t stream);

/*
 * Max-pooling of spike bits (SeqToANNContainer(MaxPool2d(k, stride, pad)),
 * models/sewresnet.py:143,203; the reference runtime's pool kernels,
 * sengine/csrc/cpp_executor.cu:77-139): in (NT, H, W) x C bits -> out (NT, OH, OW) x C
 * bits; for {0,1} values the max is the OR.  C % 32 == 0, pad <= k/2.
 */
int sengine_amd_maxpool_spikes(int32_t NT, int32_t H, int32_t W, int32_t C, int32_t k, int32_t stride, int32_t pad,
                               const uint32_t* in, uint32_t* out, hipStream_t stream);

/*
 * Head: AdaptiveAvgPool2d(1) per timestep, mean over T, Linear (models/sewresnet.py:152-153,
 * 208-210; the same values as MS-ResNet's mean over T then pool, models/msresnet.py:155-160).
 * in: integer activations as `planes` bit planes, (T*B, HW) positions x planes*C bits, or
 * (planes = 0) as integer-valued fp16 (T*B, HW, C) (Spikformer's residual stream, whose
 * reference tensor is the float sum of spikes, models/spikformer.py:148-149);
 * fc_weight (N_out, C) fp32 (nn.Linear layout), fc_bias (N_out); out (B, N_out) fp32.
 * C % 32 == 0, 0 <= planes <= 5, planes * C <= 8192.
 */
int sengine_amd_sew_head(int32_t T, int32_t B, int32_t HW, int32_t C, int32_t planes, const uint32_t* in,
                         const float* fc_weight, const float* fc_bias, int32_t N_out, float* out,
                         hipStream_t stream);

/*
 * The same head for an fp16 stream (planes = 0; other planes values behave as
 * sengine_amd_sew_head) with the per-channel sums split over up to 64 workgroups per image
 * (Spikformer's x.mean(2).mean(0) + head, models/spikformer.py:277-288, over its 3,136-token
 * grid): partial integer sums go to the caller's workspace, at least B * 64 * C int32
 * (workspace_elems), then the head adds them.  Same values as sengine_amd_sew_head (the sums
 * are exact integers).  C % 32 == 0, C <= 2048.
 */
int sengine_amd_sew_head_ws(int32_t T, int32_t B, int32_t HW, int32_t C, int32_t planes, const uint32_t* in,
                            const float* fc_weight, const float* fc_bias, int32_t N_out, float* out,
                            int32_t* workspace, int64_t workspace_elems, hipStream_t stream);

/*
 * Unfused fallback, half 1: dense Conv + folded BN, fp32 output (T*B*OH*OW, C_out).
 * Mirrors conv2d_bn_t4_kernel / conv1x1_bn_t4_kernel (conv2d_bn_if_t4.py:551-673), but
 * keeps the BN output in fp32 (the reference rounds it to fp16).
 * Requires C_in % 32 == 0, C_out % 64 == 0.
 */
int sengine_amd_dense_conv_bn(const sengine_conv_lif_desc* d, const void* data, const void* blob_values,
                              const float* bn_scale, const float* bn_bias, float* out,
                              hipStream_t stream);

/*
 * Unfused fallback, half 2: standalone multi-step neuron over T.
 * x: fp32 (T, n) with n = spatial elements per timestep; state: optional fp32 (n).
 * spikes: encoding out_enc (bits need n % 32 == 0), h_trace optional fp32 (T, n).
 * Mirrors lif_neuron_kernel / if_neuron_kernel (sengine/csrc/kernels.cuh:18-54) with the
 * reset and leak of models/neurons.py:121-146,169-184.
 */
int sengine_amd_multistep_neuron(int32_t T, int64_t n, int32_t neuron, int32_t hard_reset, float tau,
                                 float v_threshold, float v_reset, const float* x, float* state,
                                 int32_t out_enc, void* spikes, float* h_trace, hipStream_t stream);

/* Pack a dense NHWC tensor (n_pos, C) into spike bits (value != 0 -> 1); C % 32 == 0. */
int sengine_amd_pack_spikes(const void* x, int32_t x_enc, int64_t n_pos, int32_t C, uint32_t* bits,
                            hipStream_t stream);

/* Unpack spike bits (n_pos, C) into fp16 / fp32 0.0 / 1.0; C % 32 == 0. */
int sengine_amd_unpack_spikes(const uint32_t* bits, int64_t n_pos, int32_t C, void* out, int32_t out_enc,
                              hipStream_t stream);

/*
 * The fused node called with the reference runtime's own weight tensor instead of a blob:
 * the fp16 (KH, KW, C_in, C_out) weight of sengine/cuda_graph_runtime.py:233-235
 * (w_enc = SENGINE_ENC_F16, w_layout = SENGINE_WLAYOUT_HWIO; any other encoding / layout the
 * compressor accepts).  Replaces the body of the reference's per-node call()
 * (sengine/build/export_standalone.py:37-103, called at sengine/csrc/cpp_executor.cu:909-913).
 * The library keeps one 2:4 blob per (device, weight pointer, geometry): prepared on the first
 * call outside stream capture (allocation, compression, one synchronising check of the 2:4
 * pattern -- the reference executor runs three eager warm-ups before it captures,
 * cpp_executor.cu:1270-1276) and reused by later calls.  The reference reads the weight on
 * every call, so a cached blob must follow the weight's bytes: every call outside stream
 * capture reads the whole weight into a 64-bit fingerprint (one small kernel and one
 * synchronisation) and, when it differs from the fingerprint recorded at the last build --
 * the weight was updated in place, or freed and its address handed to a different weight --
 * rebuilds the blob in place before launching.  Calls inside a capture cannot synchronise:
 * they use the blob as of the last call outside capture, and a captured graph replays
 * whatever that blob holds when it runs (an eager call after a weight update refreshes it
 * for the graph too).  A weight first seen during capture returns -4; a weight that is not
 * 2:4 along C_in returns -5 (and so do captured calls after an eager call found it so).
 * sengine_amd_prepare_weight does the preparation / refresh step alone.
 * sengine_amd_release_weights frees every blob: call it only when no kernel of the library
 * is running and no captured graph that launched a raw-weight call will be replayed again
 * (the graph holds the blob's address).
 */
int sengine_amd_fused_call_raw_weight(const sengine_conv_lif_desc* d, const void* data, const void* weight,
                                      int32_t w_enc, int32_t w_layout, float* state, const float* bn_scale,
                                      const float* bn_bias, void* spikes, hipStream_t stream);
int sengine_amd_prepare_weight(const sengine_conv_lif_desc* d, const void* weight, int32_t w_enc, int32_t w_layout,
                               hipStream_t stream);
int sengine_amd_release_weights(void);

/*
 * Peak calibration on the box (the role of the reference's sengine/tuning/hw_calibrate.py:
 * 17-134, which times a memcpy and a dense fp16 GEMM).  Measurement entry points, not on
 * the operator path.
 *   calibrate_smfmac: `blocks` workgroups of 256 threads; every wave issues iters x 8
 *     back-to-back v_smfmac_f32_16x16x64_f16 from registers (32,768 dense-equivalent FLOPs
 *     each) and writes one float per thread to sink (blocks * 256 floats).
 *   calibrate_copy: streams `bytes` (a multiple of 16, 16-byte aligned buffers) from src to
 *     dst with 16-byte accesses (bytes read + bytes written of HBM traffic).
 *   calibrate_stream: the same stream in `mode` 0 (that copy), 1 (the copy with non-temporal
 *     loads and stores) or 2 (read only: bytes read; dst receives one 32-bit checksum per
 *     thread of the launch, at most bytes / 4 of it).
 */
int sengine_amd_calibrate_smfmac(int32_t blocks, int32_t iters, float* sink, hipStream_t stream);
int sengine_amd_calibrate_copy(const void* src, void* dst, int64_t bytes, hipStream_t stream);
int sengine_amd_calibrate_stream(const void* src, void* dst, int64_t bytes, int32_t mode, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SENGINE_AMD_H */
