// v7g_device.h -- device-side arithmetic shared by the gfx950 kernels.
//
// The reference kernels are AVX2 NASM with IEEE binary32 arithmetic, round to
// nearest-even, under MXCSR FTZ+DAZ (src/asm/v7_init.inc:103-108,
// SET_FTZ_DAZ src/asm/v7_core.inc:301-303): a denormal input reads as zero and
// a result still below 2^-126 after rounding becomes zero.  The library is
// built with f32 denormals flushed (-fgpu-flush-denormals-to-zero), which
// gives the same results for the operations used here (add, multiply, fma,
// division, sqrt, compare, med3, conversion to binary16); a v_cndmask select
// passes a denormal through unflushed, which no output below can observe.
// Every helper reproduces one reference instruction sequence with one
// correctly rounded gfx950 operation per x86 operation.  The library is built
// with -ffp-contract=off, so `a * b + c` stays two roundings and
// __builtin_fmaf is the only fused multiply-add; f32 division and sqrt are
// the correctly rounded expansions (hipcc's default).  The hot loops replace
// two divisions by shorter sequences that give the same bits for every input
// they can receive (rcp_rn, div127_rn below).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace v7g {

// EVAL_SIGMOID constants: src/asm/math_data.inc:16-53.
__device__ __forceinline__ float bits_f(uint32_t u) { return __builtin_bit_cast(float, u); }

// 1/d for d in [2^-126, 2^123): v_rcp_f32 (within 1 ulp) and one Newton step
// with fused multiply-adds, e = fma(-d, r, 1) (exact), r + e*r.  For every d
// in that range this equals the correctly rounded IEEE division 1.0f/d, bit
// for bit; v7g_arith_selfcheck() verifies it exhaustively on the running
// device.  Outside the range (0, Inf, subnormals) callers handle the value
// themselves.
__device__ __forceinline__ float rcp_rn(float d) {
  float r = __builtin_amdgcn_rcpf(d);
  float e = __builtin_fmaf(-d, r, 1.0f);
  return __builtin_fmaf(e, r, r);
}

// x / 127 correctly rounded, for finite x >= 127*2^-126: q0 = x*RN(1/127),
// the remainder x - 127*q0 is exact in one fma, and one more fma corrects q0.
// With denormals flushed a remainder below 2^-126 (x below about 2^-103)
// would read as zero, so x below 2^64 is divided as x*2^64 and the quotient
// scaled back by 2^-64, both exact (powers of two, normal results).  Equal to
// the IEEE division for every such x (exhaustively checked by
// v7g_arith_selfcheck()).
__device__ __forceinline__ float div127_rn(float x) {
  const bool small = x < 0x1p64f;
  const float xs = small ? x * 0x1p64f : x;
  const float inv = 1.0f / 127.0f;
  const float q0 = xs * inv;
  const float r = __builtin_fmaf(-q0, 127.0f, xs);
  const float q = __builtin_fmaf(r, inv, q0);
  return small ? q * 0x1p-64f : q;
}

// EVAL_SIGMOID, packed form (src/asm/v7_macros.inc:98-160):
//   x = clamp(-g, -80, 80); fx = x*log2e; i = rne(fx); f = fx - i;
//   p = C5; p = fma(f,p,C4) ... fma(f,p,C1); p = fma(f,p,1); e = 2^i * p;
//   sigma = 1 / (1 + e).
// The clamp is one v_med3_f32 (max then min for every non-NaN input; a NaN
// gate makes the SwiGLU product NaN on both sides whatever the clamp returns).
// 2^i * p is formed with v_ldexp_f32: the reference multiplies p by the exact
// power of two built from exponent bits, and that product is exact for the
// reachable range (|i| <= 116, p in [0.7, 1.42]), so ldexp gives the same
// bits.  1/(1+e) is rcp_rn: 1 + e lies in [1, 2^117).  The whole function
// equals the same sequence with IEEE division for all 2^32 inputs
// (v7g_arith_selfcheck()).
__device__ __forceinline__ float sigmoid_v7(float g) {
  const float log2e = 1.4426950408889634f;
  float x = __builtin_amdgcn_fmed3f(-g, -80.0f, 80.0f);
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
  return rcp_rn(e + 1.0f);
}

// SwiGLU element, src/asm/prefill_q8.inc:1159-1165: (sigma(g) * g) * u.
__device__ __forceinline__ float swiglu_v7(float g, float u) {
  float s = sigmoid_v7(g) * g;
  return s * u;
}

// The quantizer's group-max floor 127 * 2^-126 (src/asm/quantize_kernel.inc:40-41).
#define V7G_Q_FLOOR 1.4928778e-36f

// Per-group scale and reciprocal, src/asm/quantize_kernel.inc:84-89:
// wmax = max(wmax, floor); scale = wmax / 127; recip = 1 / scale.  An Inf
// group max (an Inf input) gives scale Inf and recip 0, as IEEE division does.
// wmax is a maximum of magnitudes and not NaN (a NaN group max first goes
// through vmaxss wmax, floor, which gives the floor: q8_floor below), so the
// max with the floor compares the bit patterns as unsigned integers.
__device__ __forceinline__ void q8_scale(float wmax, float &scale, float &recip) {
  const uint32_t wb = __builtin_bit_cast(uint32_t, wmax), fb = __builtin_bit_cast(uint32_t, V7G_Q_FLOOR);
  wmax = __builtin_bit_cast(float, __builtin_elementwise_max(wb, fb));
  const bool inf = wmax == __builtin_inff();
  scale = inf ? wmax : div127_rn(wmax);
  recip = inf ? 0.0f : rcp_rn(scale);
}

// One int8 code as the low byte of its two's complement, src/asm/quantize_kernel.inc:91-105
// (vmulps, vcvtps2dq, signed-saturating packs, vpmaxsb -127): rne(v)
// clamped to [-127, 127], with v = x * recip.  For finite x, |v| <= 127.00002,
// so only the lower clamp can bind; a NaN v must give -127 (x86 converts NaN
// to 0x80000000, which saturates to -128 and is raised to -127), and
// max(v, -127) returns -127 for NaN.  Adding 1.5*2^23 rounds v to an integer
// with ties to even in the low mantissa bits, whose low byte is the code.
__device__ __forceinline__ uint32_t q8_code_byte(float v) {
  v = __builtin_fmaxf(v, -127.0f);
  return __builtin_bit_cast(uint32_t, v + 12582912.0f) & 0xffu;
}
__device__ __forceinline__ int q8_code(float v) { return (int)(int8_t)q8_code_byte(v); }

__device__ __forceinline__ uint32_t pack4_codes(float4 v, float recip) {
  return q8_code_byte(v.x * recip) | (q8_code_byte(v.y * recip) << 8) | (q8_code_byte(v.z * recip) << 16) |
         (q8_code_byte(v.w * recip) << 24);
}

// The same code for any v, also beyond +-127.00002 (a group whose max lost
// elements to a NaN, below): vcvtps2dq gives 0x80000000 for NaN and for
// |v| >= 2^31, which the packs and vpmaxsb turn into -127; in range,
// rne(v) saturates to [-127, 127], and clamping before rounding gives the same.
__device__ __forceinline__ uint32_t q8_code_byte_full(float v) {
  const bool in_range = v >= -2147483648.0f && v < 2147483648.0f;
  return in_range ? q8_code_byte(__builtin_amdgcn_fmed3f(v, -127.0f, 127.0f)) : 0x81u;
}
__device__ __forceinline__ uint32_t pack4_codes_full(float4 v, float recip) {
  return q8_code_byte_full(v.x * recip) | (q8_code_byte_full(v.y * recip) << 8) |
         (q8_code_byte_full(v.z * recip) << 16) | (q8_code_byte_full(v.w * recip) << 24);
}


// The fast path of a group whose lanes hold only finite values: the group max
// is finite, so q8_scale's Inf case cannot arise and every code's v lies in
// [-127.00003, 127.00003], where the magic-number rounding needs no clamp.
__device__ __forceinline__ void q8_scale_finite(float wmax, float &scale, float &recip) {
  const uint32_t wb = __builtin_bit_cast(uint32_t, wmax), fb = __builtin_bit_cast(uint32_t, V7G_Q_FLOOR);
  scale = div127_rn(__builtin_bit_cast(float, __builtin_elementwise_max(wb, fb)));
  recip = rcp_rn(scale);
}
__device__ __forceinline__ uint32_t q8_code_byte_finite(float v) {
  return __builtin_bit_cast(uint32_t, v + 12582912.0f) & 0xffu;
}
__device__ __forceinline__ uint32_t pack4_codes_finite(float4 v, float recip) {
  return q8_code_byte_finite(v.x * recip) | (q8_code_byte_finite(v.y * recip) << 8) |
         (q8_code_byte_finite(v.z * recip) << 16) | (q8_code_byte_finite(v.w * recip) << 24);
}
// vmaxps / vmaxss a, b: a > b ? a : b, the second operand when either is NaN.
__device__ __forceinline__ float vmax_x86(float a, float b) { return (a > b) ? a : b; }

// vmaxss wmax, floor (quantize_kernel.inc:84) for a group max that may be NaN.
__device__ __forceinline__ float q8_floor(float wmax) { return vmax_x86(wmax, V7G_Q_FLOOR); }

// binary32 -> binary16 with round to nearest even (v_cvt_f16_f32 in the
// default rounding mode, binary16 subnormals kept), the conversion of the
// reference's vcvtps2ph with imm 0 (src/asm/kv_f16c.inc:5-7); finite inputs
// and infinities give identical bits, NaN stays NaN.  v7g_arith_selfcheck()
// compares it with a software rounding over every binary32 pattern.
__device__ __forceinline__ uint32_t f16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}
// Four floats as four binary16 values in two dwords (little-endian order).
__device__ __forceinline__ uint2 pack4_f16(float4 v) {
  return make_uint2(f16_bits(v.x) | (f16_bits(v.y) << 16), f16_bits(v.z) | (f16_bits(v.w) << 16));
}

// Streaming (nontemporal) loads and stores for activations that each kernel
// reads or writes exactly once.  They keep the stream out of L2 and the
// Infinity Cache (MALL): the reused lines (RoPE tables, norm weights, table
// scales) stay resident, and a kernel leaves no dirty lines behind for the
// next kernel of the chain to write back.  Measured on MI355X over the whole
// per-layer chain, every kernel is fastest with streaming loads and stores,
// except that the embedding gather writes its output rows with ordinary
// stores (they stay cached for the layer that reads them next).
typedef float v7g_f4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_stream4(const float *p) {
  v7g_f4 a = __builtin_nontemporal_load(reinterpret_cast<const v7g_f4 *>(p));
  return make_float4(a.x, a.y, a.z, a.w);
}
__device__ __forceinline__ void st_stream4(float *p, float4 v) {
  v7g_f4 a = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(a, reinterpret_cast<v7g_f4 *>(p));
}
__device__ __forceinline__ uint32_t ld_stream_u32(const uint32_t *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_stream_u32(uint32_t *p, uint32_t v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void st_stream_f32(float *p, float v) { __builtin_nontemporal_store(v, p); }
typedef unsigned int v7g_u2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void st_stream_u2(uint32_t *p, uint2 v) {
  v7g_u2 a = {v.x, v.y};
  __builtin_nontemporal_store(a, reinterpret_cast<v7g_u2 *>(p));
}

// DPP lane exchanges inside a 16-lane row (gfx9 encodings).
enum : int {
  DPP_QUAD_XOR1 = 0xB1,         // quad_perm [1,0,3,2]
  DPP_QUAD_XOR2 = 0x4E,         // quad_perm [2,3,0,1]
  DPP_ROW_HALF_MIRROR = 0x141,  // lane i <-> 7-i within each 8 lanes
  DPP_ROW_MIRROR = 0x140,       // lane i <-> 15-i within each 16 lanes
};

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return __builtin_elementwise_max(a, b); }

// Max over aligned groups of 8 lanes of non-negative, non-NaN floats: their
// bit patterns order as unsigned integers do, so each step is one
// v_max_u32 with a DPP operand (order-free, and no NaN quieting).
__device__ __forceinline__ float group8_max(float f) {
  uint32_t v = __builtin_bit_cast(uint32_t, f);
  v = umax(v, dpp_u<DPP_QUAD_XOR1>(v));
  v = umax(v, dpp_u<DPP_QUAD_XOR2>(v));
  v = umax(v, dpp_u<DPP_ROW_HALF_MIRROR>(v));
  return __builtin_bit_cast(float, v);
}

// The same over aligned groups of 16 lanes.
__device__ __forceinline__ float group16_max(float f) {
  uint32_t v = __builtin_bit_cast(uint32_t, group8_max(f));
  v = umax(v, dpp_u<DPP_ROW_MIRROR>(v));
  return __builtin_bit_cast(float, v);
}

// Lane exchange by xor inside the wave (ds_bpermute); exact pairing for the
// ordered reductions, where every lane must end with bit-identical sums.
__device__ __forceinline__ float xor_f(float v, int mask) {
  int lane = __lane_id();
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __builtin_bit_cast(int, v)));
}

// |x|, |y|, |z|, |w| reduced with v_maximum3_f32, which propagates NaN: the
// lane's share of a group max, NaN exactly when one of its elements is NaN.
__device__ __forceinline__ float lane_absmax4(float4 v) {
  return __builtin_elementwise_maximum(
      __builtin_elementwise_maximum(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
      __builtin_elementwise_maximum(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
}

// True for every lane of the wave when some lane's value is NaN or infinite.
__device__ __forceinline__ bool wave_any_nonfinite(float m) {
  return __builtin_amdgcn_ballot_w64(!(m < __builtin_inff())) != 0;
}

// One level of an ordered max tree across lanes l and l ^ MASK: the lane with
// the bit clear supplies the first operand, so both lanes get the same value.
template <int MASK>
__device__ __forceinline__ float tree_max_step(float a) {
  const float o = xor_f(a, MASK);
  return (__lane_id() & MASK) ? vmax_x86(o, a) : vmax_x86(a, o);
}

// Group absmax with the reference's vmaxps tree and operand order
// (src/asm/quantize_kernel.inc:62-83, src/asm/rmsnorm_quantize_kernel.inc:158-186).
// Without NaN it is the plain maximum; with NaN, the operand order decides
// whether the NaN reaches wmax (which the floor then replaces) or drops out
// together with the values it was paired with.  The group's GS/4 lanes hold 4
// consecutive elements each: element e = 4l + k is lane i = e % 8 = 4(l&1) + k
// of YMM vector j = e / 8 = l/2.  The per-lane levels pair vectors j^1, j^2,
// j^4 (lanes l^2, l^4, l^8; GS = 32 stops after j^2), vextractf128 pairs lane
// i with i+4 (lanes l^1), and vmovhlps / vmovshdup pair components k with k+2,
// then 0 with 1, inside the lane.  Every lane of the group returns the value.
template <int GS>
__device__ __forceinline__ float group_absmax_tree(float4 v) {
  float a[4] = {__builtin_fabsf(v.x), __builtin_fabsf(v.y), __builtin_fabsf(v.z), __builtin_fabsf(v.w)};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    a[k] = tree_max_step<2>(a[k]);
    a[k] = tree_max_step<4>(a[k]);
    if constexpr (GS == 64) a[k] = tree_max_step<8>(a[k]);
    a[k] = tree_max_step<1>(a[k]);
  }
  return vmax_x86(vmax_x86(a[0], a[2]), vmax_x86(a[1], a[3]));
}

// The same tree when each lane of the group holds 16 consecutive elements
// (YMM vectors 2L and 2L+1 of the group on lane L; GS/16 lanes per group,
// aligned in the wave): vectors 2L, 2L+1 pair inside the lane, the next
// levels pair lanes L^1 (and L^2 for 64), lower lane first; then lanes i with
// i+4 of the 8-float vector (vextractf128), k with k+2 (vmovhlps), 0 with 1
// (vmovshdup).  Every lane of the group returns the value.
template <int GS>
__device__ __forceinline__ float group_absmax_tree16(const float (&a)[16]) {
  float m[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) m[i] = vmax_x86(__builtin_fabsf(a[i]), __builtin_fabsf(a[8 + i]));
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    m[i] = tree_max_step<1>(m[i]);
    if constexpr (GS == 64) m[i] = tree_max_step<2>(m[i]);
  }
  float r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = vmax_x86(m[i], m[i + 4]);
  return vmax_x86(vmax_x86(r[0], r[2]), vmax_x86(r[1], r[3]));
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
