// v7g_device.h -- device-side arithmetic shared by the gfx950 kernels.
//
// The reference kernels are AVX2 NASM with IEEE binary32 arithmetic, round to
// nearest-even.  Every helper below reproduces one reference instruction
// sequence with one correctly rounded gfx950 operation per x86 operation.
// The library is built with -ffp-contract=off, so `a * b + c` stays two
// roundings and __builtin_fmaf is the only fused multiply-add; f32 division
// and sqrt are the correctly rounded expansions (hipcc's default).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace v7g {

// EVAL_SIGMOID constants: src/asm/math_data.inc:16-53.
__device__ __forceinline__ float bits_f(uint32_t u) { return __builtin_bit_cast(float, u); }

// EVAL_SIGMOID, packed form (src/asm/v7_macros.inc:98-160):
//   x = clamp(-g, -80, 80); fx = x*log2e; i = rne(fx); f = fx - i;
//   p = C5; p = fma(f,p,C4) ... fma(f,p,C1); p = fma(f,p,1); e = 2^i * p;
//   sigma = 1 / (1 + e).
// 2^i * p is formed with v_ldexp_f32: the reference multiplies p by the
// exact power of two built from exponent bits, and that product is exact for
// the reachable range (|i| <= 116, p in [0.7, 1.42]), so ldexp gives the same
// bits in one instruction.  The clamp uses max/min: identical to x86
// vmaxps/vminps for every non-NaN input; a NaN gate makes the SwiGLU product
// NaN on both sides whatever the clamp returns.
__device__ __forceinline__ float sigmoid_v7(float g) {
  const float log2e = 1.4426950408889634f;
  float x = -g;
  x = __builtin_fmaxf(x, -80.0f);
  x = __builtin_fminf(x, 80.0f);
  float fx = x * log2e;
  float ip = __builtin_rintf(fx);
  float fp = fx - ip;
  float p = bits_f(0x3AADD303u);
  p = __builtin_fmaf(fp, p, bits_f(0x3C1E7411u));
  p = __builtin_fmaf(fp, p, bits_f(0x3D635B9Bu));
  p = __builtin_fmaf(fp, p, bits_f(0x3E75FCE0u));
  p = __builtin_fmaf(fp, p, bits_f(0x3F317215u));
  p = __builtin_fmaf(fp, p, 1.0f);
  float e = __builtin_ldexpf(p, (int)ip);
  float d = e + 1.0f;
  return 1.0f / d;
}

// SwiGLU element, src/asm/prefill_q8.inc:1159-1165: (sigma(g) * g) * u.
__device__ __forceinline__ float swiglu_v7(float g, float u) {
  float s = sigmoid_v7(g) * g;
  return s * u;
}

// The quantizer's group-max floor 127 * 2^-126 (src/asm/quantize_kernel.inc:40-41).
#define V7G_Q_FLOOR 1.4928778e-36f

// Per-group scale and reciprocal, src/asm/quantize_kernel.inc:84-89:
// wmax = max(wmax, floor); scale = wmax / 127; recip = 1 / scale.
__device__ __forceinline__ void q8_scale(float wmax, float &scale, float &recip) {
  wmax = (wmax > V7G_Q_FLOOR) ? wmax : V7G_Q_FLOOR;
  scale = wmax / 127.0f;
  recip = 1.0f / scale;
}

// One int8 code, src/asm/quantize_kernel.inc:91-105 (vmulps, vcvtps2dq,
// signed-saturating packs, vpmaxsb -127): rne(x * recip) clamped to
// [-127, 127]; a NaN product gives -127 (x86 converts NaN to 0x80000000,
// which saturates to -128 and is raised to -127).  fmaxf returns the non-NaN
// operand, so NaN lands on -127 here too.  |x * recip| <= 127.00002 for every
// finite input, so the out-of-int32-range case of vcvtps2dq is unreachable.
__device__ __forceinline__ int q8_code(float v) {
  float r = __builtin_rintf(v);
  r = __builtin_fmaxf(r, -127.0f);
  r = __builtin_fminf(r, 127.0f);
  return (int)r;
}

__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
         ((uint32_t)(d & 0xff) << 24);
}

// DPP lane exchanges inside a 16-lane row (gfx9 encodings).
enum : int {
  DPP_QUAD_XOR1 = 0xB1,         // quad_perm [1,0,3,2]
  DPP_QUAD_XOR2 = 0x4E,         // quad_perm [2,3,0,1]
  DPP_ROW_HALF_MIRROR = 0x141,  // lane i <-> 7-i within each 8 lanes
  DPP_ROW_MIRROR = 0x140,       // lane i <-> 15-i within each 16 lanes
};

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// max over aligned groups of 8 lanes (order-free for non-NaN input).
__device__ __forceinline__ float group8_max(float v) {
  v = __builtin_fmaxf(v, dpp_f<DPP_QUAD_XOR1>(v));
  v = __builtin_fmaxf(v, dpp_f<DPP_QUAD_XOR2>(v));
  v = __builtin_fmaxf(v, dpp_f<DPP_ROW_HALF_MIRROR>(v));
  return v;
}

// max over aligned groups of 16 lanes.
__device__ __forceinline__ float group16_max(float v) {
  v = group8_max(v);
  v = __builtin_fmaxf(v, dpp_f<DPP_ROW_MIRROR>(v));
  return v;
}

// Lane exchange by xor inside the wave (ds_bpermute); exact pairing for the
// ordered reductions, where every lane must end with bit-identical sums.
__device__ __forceinline__ float xor_f(float v, int mask) {
  int lane = __lane_id();
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __builtin_bit_cast(int, v)));
}

// COMPUTE_RMS_SCALE, src/asm/v7_macros.inc:348-354: 1 / sqrt(sumsq/n + eps),
// four correctly rounded operations.
__device__ __forceinline__ float rms_scale(float sumsq, float n, float eps) {
  float mean = sumsq / n;
  float val = mean + eps;
  float root = __builtin_sqrtf(val);
  return 1.0f / root;
}

}  // namespace v7g
