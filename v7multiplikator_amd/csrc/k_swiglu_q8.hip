// k_swiglu_q8.hip -- elementwise SwiGLU, SwiGLU -> Q8 and Q8 block quantization, gfx950.
//
// References:
//   .pq_ffn_silu (src/asm/prefill_q8.inc:1159-1166): out = (sigmoid(g)*g)*u
//     with EVAL_SIGMOID (src/asm/v7_macros.inc:98-160);
//   v7d_quantize / v7s_quantize_chunk (src/asm/utility_dispatch.inc:108-212,
//     src/asm/quantize_kernel.inc:44-159): per group of GS floats,
//     wmax = max|x| floored at 127*2^-126, scale = wmax/127 (stored),
//     recip = 1/scale, code = sat(rne(x*recip)) raised to -127; a partial
//     tail group uses the same arithmetic.
//   The SwiGLU -> Q8 chain (src/asm/prefill_q8.inc:1154-1183) quantizes the
//   SwiGLU row; here the SwiGLU values never leave registers.
// The reference group size is 64 (src/asm/v7_core.inc:120); GS is a template
// parameter so 32-element blocks use the same algorithm.
//
// Vector layout: lane owns 4 consecutive floats (dwordx4 loads of gate and up
// or x), GS/4 consecutive lanes form one group, the group max is a DPP
// butterfly inside 8 or 16 lanes, each lane stores its 4 codes as one dword,
// and the first lane of the group stores the scale.
#include "v7g_device.h"
#include "v7g_internal.h"

namespace v7g {

constexpr int kSwigluU = 4;  // float4 chunks per thread in flight
constexpr int kQuantU = 4;

__global__ __launch_bounds__(256) void swiglu_f32_kernel(float *out, const float *gate, const float *up, long long n4) {
  const long long base = (long long)blockIdx.x * (256 * kSwigluU) + threadIdx.x;
  const float4 *g4 = reinterpret_cast<const float4 *>(gate);
  const float4 *u4 = reinterpret_cast<const float4 *>(up);
  float4 *o4 = reinterpret_cast<float4 *>(out);
  float4 g[kSwigluU], u[kSwigluU];
#pragma unroll
  for (int k = 0; k < kSwigluU; ++k) {
    long long c = base + k * 256;
    if (c < n4) {
      g[k] = g4[c];
      u[k] = u4[c];
    }
  }
#pragma unroll
  for (int k = 0; k < kSwigluU; ++k) {
    long long c = base + k * 256;
    if (c < n4)
      o4[c] = make_float4(swiglu_v7(g[k].x, u[k].x), swiglu_v7(g[k].y, u[k].y), swiglu_v7(g[k].z, u[k].z),
                          swiglu_v7(g[k].w, u[k].w));
  }
}

// Elements n - n%4 .. n-1 (fewer than 4), one thread each.
__global__ void swiglu_f32_tail_kernel(float *out, const float *gate, const float *up, long long start, long long n) {
  long long i = start + threadIdx.x;
  if (i < n) out[i] = swiglu_v7(gate[i], up[i]);
}

void launch_swiglu_f32(float *out, const float *gate, const float *up, long long n, hipStream_t stream) {
  long long n4 = n / 4;
  if (n4 > 0) {
    long long blocks = (n4 + 256 * kSwigluU - 1) / (256 * kSwigluU);
    hipLaunchKernelGGL(swiglu_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, out, gate, up, n4);
  }
  if (n % 4)
    hipLaunchKernelGGL(swiglu_f32_tail_kernel, dim3(1), dim3(4), 0, stream, out, gate, up, n4 * 4, n);
}

// Flat path: every row length is a multiple of GS, so groups tile the flat
// array and group g covers elements [g*GS, (g+1)*GS).
template <int GS, bool SWIGLU>
__global__ __launch_bounds__(256) void quantize_q8_flat_kernel(int8_t *__restrict__ out_q, float *__restrict__ out_s,
                                                               const float *__restrict__ x,
                                                               const float *__restrict__ gate,
                                                               const float *__restrict__ up, long long n4) {
  constexpr int LPG = GS / 4;  // lanes per group
  const long long base = (long long)blockIdx.x * (256 * kQuantU) + threadIdx.x;
  float4 v[kQuantU];
#pragma unroll
  for (int k = 0; k < kQuantU; ++k) {
    long long c = base + k * 256;
    if (c < n4) {
      if constexpr (SWIGLU) {
        float4 g = reinterpret_cast<const float4 *>(gate)[c];
        float4 u = reinterpret_cast<const float4 *>(up)[c];
        v[k] = make_float4(g.x, g.y, g.z, g.w);
        v[k].x = swiglu_v7(g.x, u.x);
        v[k].y = swiglu_v7(g.y, u.y);
        v[k].z = swiglu_v7(g.z, u.z);
        v[k].w = swiglu_v7(g.w, u.w);
      } else {
        v[k] = reinterpret_cast<const float4 *>(x)[c];
      }
    } else {
      v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
#pragma unroll
  for (int k = 0; k < kQuantU; ++k) {
    const long long c = base + k * 256;
    float m = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v[k].x), __builtin_fabsf(v[k].y)),
                              __builtin_fmaxf(__builtin_fabsf(v[k].z), __builtin_fabsf(v[k].w)));
    m = (LPG == 8) ? group8_max(m) : group16_max(m);
    float scale, recip;
    q8_scale(m, scale, recip);
    if (c < n4) {
      uint32_t packed = pack4_i8(q8_code(v[k].x * recip), q8_code(v[k].y * recip), q8_code(v[k].z * recip),
                                 q8_code(v[k].w * recip));
      reinterpret_cast<uint32_t *>(out_q)[c] = packed;
      if ((threadIdx.x & (LPG - 1)) == 0) out_s[c / LPG] = scale;
    }
  }
}

// General path: any row length, any GS in [4, 256]; one thread per group,
// scalar loads.  A partial last group of a row takes the reference's scalar
// tail arithmetic (quantize_kernel.inc:119-152), value-identical to the
// vector path for every non-NaN input.
template <bool SWIGLU>
__global__ __launch_bounds__(256) void quantize_q8_generic_kernel(int8_t *out_q, float *out_s, const float *x,
                                                                  const float *gate, const float *up, int rows,
                                                                  int row_len, int gs) {
  const int spr = (row_len + gs - 1) / gs;
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long long)rows * spr) return;
  const long long r = gid / spr;
  const int g = (int)(gid - r * spr);
  const long long start = r * row_len + (long long)g * gs;
  const int len = min(gs, row_len - g * gs);
  float wmax = 0.0f;
  for (int i = 0; i < len; ++i) {
    float v = SWIGLU ? swiglu_v7(gate[start + i], up[start + i]) : x[start + i];
    float a = __builtin_fabsf(v);
    wmax = (a > wmax) ? a : wmax;
  }
  float scale, recip;
  q8_scale(wmax, scale, recip);
  out_s[r * spr + g] = scale;
  for (int i = 0; i < len; ++i) {
    float v = SWIGLU ? swiglu_v7(gate[start + i], up[start + i]) : x[start + i];
    out_q[start + i] = (int8_t)q8_code(v * recip);
  }
}

template <int GS>
static void launch_flat(int8_t *out_q, float *out_s, const float *x, const float *gate, const float *up, long long n,
                        hipStream_t stream) {
  long long n4 = n / 4;
  long long blocks = (n4 + 256 * kQuantU - 1) / (256 * kQuantU);
  if (gate)
    hipLaunchKernelGGL((quantize_q8_flat_kernel<GS, true>), dim3((unsigned)blocks), dim3(256), 0, stream, out_q, out_s,
                       x, gate, up, n4);
  else
    hipLaunchKernelGGL((quantize_q8_flat_kernel<GS, false>), dim3((unsigned)blocks), dim3(256), 0, stream, out_q,
                       out_s, x, gate, up, n4);
}

static bool aligned(const void *p, size_t a) { return p == nullptr || ((uintptr_t)p % a) == 0; }

void launch_quantize_q8(int8_t *out_q, float *out_s, const float *x, const float *gate, const float *up, int rows,
                        int row_len, int gs, hipStream_t stream) {
  const long long n = (long long)rows * row_len;
  const bool flat = (gs == 32 || gs == 64) && row_len % gs == 0 && aligned(out_q, 4) && aligned(x, 16) &&
                    aligned(gate, 16) && aligned(up, 16) && n / 4 < (1LL << 40);
  if (flat) {
    if (gs == 32)
      launch_flat<32>(out_q, out_s, x, gate, up, n, stream);
    else
      launch_flat<64>(out_q, out_s, x, gate, up, n, stream);
    return;
  }
  const long long groups = (long long)rows * ((row_len + gs - 1) / gs);
  const unsigned blocks = (unsigned)((groups + 255) / 256);
  if (gate)
    hipLaunchKernelGGL((quantize_q8_generic_kernel<true>), dim3(blocks), dim3(256), 0, stream, out_q, out_s, x, gate,
                       up, rows, row_len, gs);
  else
    hipLaunchKernelGGL((quantize_q8_generic_kernel<false>), dim3(blocks), dim3(256), 0, stream, out_q, out_s, x, gate,
                       up, rows, row_len, gs);
}

}  // namespace v7g
