// Shared device helpers for the gfx950 kernels of sengine_amd.
//
// Operand layouts of the CDNA4 matrix instructions used here (measured on the
// MI355X with a known-answer probe, not taken from any document):
//   v_smfmac_f32_16x16x64_f16  D(16x16) += A(16x64, 2:4 sparse along k) * B(64x16)
//     A lane l : row l%16, 8 compressed fp16 values j=0..7; value j sits in 4-group
//                j/2 of k-range [16*(l/16), 16*(l/16)+16) at position idx[2j+1:2j]
//                (idx = 16-bit metadata selected by ABID).
//     B lane l : column l%16, 16 fp16 values; value j<8 is k = 8*(l/16)+j,
//                value j>=8 is k = 32 + 8*(l/16) + (j-8).
//     D lane l : value i is row 4*(l/16)+i, column l%16.
//   v_mfma_f32_16x16x32_f16    (dense)
//     A lane l : row l%16, k = 8*(l/16)+j;  B lane l: k = 8*(l/16)+j, column l%16.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sengine_amd.h"

namespace sengine {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half16_t __attribute__((ext_vector_type(16)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x8_t __attribute__((ext_vector_type(8)));

// Fourth dword of a raw buffer resource on gfx9 parts (untyped 32-bit data, no swizzle):
// loads through it are bounds-checked against num_records bytes and return 0 beyond.
constexpr int kBufferDword3 = 0x00020000;

// Spike value fed to the matrix cores for a set bit: fp16 2.0 (0x4000) is a single
// set bit, so expansion is one shift + one mask per register.  The factor 2 is exact
// and folded into the epilogue scale.
constexpr float kBitSpikeValue = 2.0f;

// Spread 16 spike bits x (bit j -> B value j) into a 16-value fp16 B fragment.
// X = x | x<<15 holds bit j at position j and at 15+j; shifting left by 14-2j moves
// bit 2j to 14 and bit 2j+1 (upper copy) to 30, the exponent MSB of each half.
__device__ __forceinline__ half16_t expand_bits16(uint32_t x) {
  const uint32_t X = x | (x << 15);
  u32x8_t r;
  r[0] = (X << 14) & 0x40004000u;
  r[1] = (X << 12) & 0x40004000u;
  r[2] = (X << 10) & 0x40004000u;
  r[3] = (X << 8) & 0x40004000u;
  r[4] = (X << 6) & 0x40004000u;
  r[5] = (X << 4) & 0x40004000u;
  r[6] = (X << 2) & 0x40004000u;
  r[7] = X & 0x40004000u;
  return __builtin_bit_cast(half16_t, r);
}

// Same for 8 bits -> 8 fp16 values (dense 16x16x32 B fragment).  X is hidden from the
// optimizer: for an 8-bit x it would rewrite each X << k as a multiplication by a 30-bit
// constant, which runs on the quarter-rate integer multiplier instead of two full-rate ops.
__device__ __forceinline__ half8_t expand_bits8(uint32_t x) {
  uint32_t X = x | (x << 15);
  asm("" : "+v"(X));
  u32x4_t r;
  r[0] = (X << 14) & 0x40004000u;
  r[1] = (X << 12) & 0x40004000u;
  r[2] = (X << 10) & 0x40004000u;
  r[3] = (X << 8) & 0x40004000u;
  return __builtin_bit_cast(half8_t, r);
}

__device__ __forceinline__ half16_t concat8(half8_t lo, half8_t hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
}

// Neuron parameters as the kernels consume them.  The recurrences follow
// models/neurons.py:121-146 (LIF) and :169-184 (IF) operation by operation:
//   LIF: v = v*(1 - 1/tau) + x/tau ; IF: v = v + x
//   spike = (v - v_th) >= 0  (== v >= v_th for finite IEEE values)
//   hard reset: v = spike ? v_reset : v ; soft reset: v = spike ? v - v_th : v
// When 1/tau is a power of two (tau = 2 in every reference config) the division and
// the decay product are exact, so x/tau is folded into the BN scale/bias and the
// charge becomes one fused multiply-add with the same rounding as the two-step form.
struct NeuronParams {
  int neuron;      // SENGINE_NEURON_LIF / IF
  int hard_reset;
  int pow2;        // 1/tau is an exact power of two (LIF only)
  float tau;       // fp32 tau (division operand)
  float decay;     // fp32(1 - 1/tau), rounded like the reference's python scalar
  float rtau;      // 1/tau when pow2
  float vth, vreset;
};

constexpr int kMaxPlanes = 5;  // bit planes of an integer activation: values up to 31 (Spikformer's residual stream)

// SEW 'ADD' connection fused into a fused layer's output (models/sewresnet.py:58-59; the
// reference's conv2d_bn_if_add_t4_kernel, sengine/kernels/conv2d_bn_if_t4.py:813-911):
// out = spike + residual, integer-valued.  Integer activations are stored as bit planes
// interleaved per position: an activation with P planes is an NHWC spike-bit tensor of P*C
// channels, plane p holding bit p of every channel's value (channel c of plane p is channel
// p*C + c).  res == nullptr: plain spike output.
struct SewAdd {
  const uint8_t* res;
  int res_planes;  // planes of the residual (1..3)
  int out_planes;  // planes written (>= res_planes; the caller sizes it so no carry is lost)
  int pix_ch;      // channels per output pixel: planes interleave per pixel, (pixel, plane, c)
  // Membrane-shortcut form (MS-ResNet): y = BN output + real_res (when given) is stored to
  // real_out (fp32, the layout of the traces) and the neuron runs on y.
  const float* real_res;
  float* real_out;
  // fp16 residual stream (the reference add kernel's own form): with fp16 output the stored
  // value is spike + res16 at the same (t, position, channel); res == nullptr then.
  const _Float16* res16;
  // Channel-split spike-bit output (no residual): channel c goes to plane c / split_c, channel
  // c % split_c, planes split_bytes apart, each a (rows, split_c) bit matrix; 0 = one plane.
  int split_c = 0;
  int64_t split_bytes = 0;
};

// One charge step: returns the charged membrane h given the previous membrane v and
// the input x.  xf is x/tau already folded (pow2 LIF) or the raw BN output.
__device__ __forceinline__ float neuron_charge(const NeuronParams& np, float v, float xf) {
  if (np.neuron == SENGINE_NEURON_IF) return __fadd_rn(v, xf);
  if (np.pow2) return __builtin_fmaf(v, np.decay, xf);  // v*decay exact => single rounding
  return __fadd_rn(__fmul_rn(v, np.decay), __fdiv_rn(xf, np.tau));
}

__device__ __forceinline__ float neuron_reset(const NeuronParams& np, float h, bool spike) {
  if (np.hard_reset) return spike ? np.vreset : h;
  return spike ? __fsub_rn(h, np.vth) : h;
}

}  // namespace sengine
