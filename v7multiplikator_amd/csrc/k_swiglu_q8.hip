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
// Vector layout: lane owns 4 consecutive floats (streaming dwordx4 loads of
// gate and up, or x), GS/4 consecutive lanes form one group, the group max is
// a DPP butterfly inside 8 or 16 lanes (the reference's ordered vmaxps tree in
// a wave that holds a NaN or an Inf), each lane stores its 4 codes as one
// dword, and the first lane of the group stores the scale.  The divisions of
// the reference (sigmoid's 1/(1+e), wmax/127, 1/scale) are the shorter
// sequences of v7g_device.h that give the same bits for every reachable input.
#include "v7g_device.h"
#include "v7g_internal.h"

namespace v7g {

// One float4 chunk per thread and a grid that covers the array once, with no
// loop: a thread's loads are issued together, many waves keep them in flight,
// and a wave carries no loop or grid-stride bookkeeping (a grid-stride loop
// cost the SwiGLU -> Q8 kernel 20 vector instructions per wave and about 2%
// of its time).  Addresses are the block's uniform base plus a 32-bit lane
// offset (scalar base, vector offset loads).  The element counts the entries
// accept (below 2^40) keep the grid below 2^31 blocks.
constexpr unsigned kStreamBlock = 256;

static unsigned stream_blocks(long long n4) { return (unsigned)((n4 + kStreamBlock - 1) / kStreamBlock); }

__global__ __launch_bounds__(kStreamBlock) void swiglu_f32_kernel(float *out, const float *gate, const float *up,
                                                                  long long n4) {
  const long long c0 = (long long)blockIdx.x * kStreamBlock;  // the block's first chunk (uniform)
  if (c0 + threadIdx.x >= n4) return;
  const unsigned t4 = 4u * threadIdx.x;
  const float4 g = ld_stream4((gate + 4 * c0) + t4);
  const float4 u = ld_stream4((up + 4 * c0) + t4);
  st_stream4((out + 4 * c0) + t4,
             make_float4(swiglu_v7(g.x, u.x), swiglu_v7(g.y, u.y), swiglu_v7(g.z, u.z), swiglu_v7(g.w, u.w)));
}

// Elements n - n%4 .. n-1 (fewer than 4), one thread each.
__global__ void swiglu_f32_tail_kernel(float *out, const float *gate, const float *up, long long start, long long n) {
  long long i = start + threadIdx.x;
  if (i < n) out[i] = swiglu_v7(gate[i], up[i]);
}

void launch_swiglu_f32(float *out, const float *gate, const float *up, long long n, hipStream_t stream) {
  long long n4 = n / 4;
  if (n4 > 0)
    enqueue(swiglu_f32_kernel, dim3(stream_blocks(n4)), dim3(kStreamBlock), 0, stream, out, gate, up, n4);
  if (n % 4)
    enqueue(swiglu_f32_tail_kernel, dim3(1), dim3(4), 0, stream, out, gate, up, n4 * 4, n);
}

// v7s_add_inplace (src/asm/add_kernel.inc:26-49): x = x + y, one vaddps per
// element; streamed like the kernels above.
__global__ __launch_bounds__(kStreamBlock) void add_inplace_kernel(float *x, const float *y, long long n4) {
  const long long c0 = (long long)blockIdx.x * kStreamBlock;
  if (c0 + threadIdx.x >= n4) return;
  const unsigned t4 = 4u * threadIdx.x;
  const float4 a = ld_stream4((x + 4 * c0) + t4);
  const float4 b = ld_stream4((y + 4 * c0) + t4);
  st_stream4((x + 4 * c0) + t4, make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w));
}

__global__ void add_inplace_tail_kernel(float *x, const float *y, long long start, long long n) {
  long long i = start + threadIdx.x;
  if (i < n) x[i] = x[i] + y[i];
}

void launch_add_inplace(float *x, const float *y, long long n, hipStream_t stream) {
  long long n4 = n / 4;
  if (n4 > 0)
    enqueue(add_inplace_kernel, dim3(stream_blocks(n4)), dim3(kStreamBlock), 0, stream, x, y, n4);
  if (n % 4) enqueue(add_inplace_tail_kernel, dim3(1), dim3(4), 0, stream, x, y, n4 * 4, n);
}

// Flat path: every row length is a multiple of GS, so groups tile the flat
// array and group g covers elements [g*GS, (g+1)*GS).  GS/4 consecutive lanes
// hold one group (8 or 16 lanes, aligned inside the wave, so a group never
// straddles two waves or two loop iterations); their max is a DPP butterfly.
template <int GS, bool SWIGLU>
__global__ __launch_bounds__(kStreamBlock) void quantize_q8_flat_kernel(int8_t *__restrict__ out_q,
                                                                        float *__restrict__ out_s,
                                                                        const float *__restrict__ x,
                                                                        const float *__restrict__ gate,
                                                                        const float *__restrict__ up, long long n4) {
  constexpr int LPG = GS / 4;  // lanes per group
  {
    const long long c0 = (long long)blockIdx.x * kStreamBlock;  // the block's first chunk (uniform)
    const long long c = c0 + threadIdx.x;
    if (c >= n4) return;
    const unsigned t4 = 4u * threadIdx.x;
    float4 v;
    if constexpr (SWIGLU) {
      const float4 g = ld_stream4((gate + 4 * c0) + t4);
      const float4 u = ld_stream4((up + 4 * c0) + t4);
      v = make_float4(swiglu_v7(g.x, u.x), swiglu_v7(g.y, u.y), swiglu_v7(g.z, u.z), swiglu_v7(g.w, u.w));
    } else {
      v = ld_stream4((x + 4 * c0) + t4);
    }
    // absmax: without NaN the vmaxps tree is a plain maximum, a DPP butterfly
    // here; a wave holding a NaN takes the reference's ordered tree instead,
    // and one holding an Inf the same general path (scale Inf, codes 0 / -127).
    float m = lane_absmax4(v);
    float scale, recip;
    uint32_t codes;
    if (!wave_any_nonfinite(m)) {
      m = (LPG == 8) ? group8_max(m) : group16_max(m);
      q8_scale_finite(m, scale, recip);
      codes = pack4_codes_finite(v, recip);
    } else {
      q8_scale(q8_floor(group_absmax_tree<GS>(v)), scale, recip);
      codes = pack4_codes_full(v, recip);
    }
    st_stream_u32((reinterpret_cast<uint32_t *>(out_q) + c0) + threadIdx.x, codes);
    if ((threadIdx.x & (LPG - 1)) == 0) st_stream_f32((out_s + c0 / LPG) + threadIdx.x / LPG, scale);
  }
}

// General path: any row length, any GS in [1, 4096]; one thread per group,
// scalar loads.  A full group of 32 or 64 takes the reference's ordered vmaxps
// tree; any other group, and a partial last group of a row, scans in order as
// the reference's scalar tail does (quantize_kernel.inc:119-152: vmaxss |x|,
// wmax drops a NaN element), which for non-NaN input is the same maximum.
// The codes of a tail group cannot leave [-127.00002, 127.00002] except as
// NaN, where the tail's vmaxss/vminss/vcvtss2si and the vector conversion both
// give -127, so one conversion serves both.
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
  auto value = [&](int i) { return SWIGLU ? swiglu_v7(gate[start + i], up[start + i]) : x[start + i]; };
  float wmax = 0.0f;
  if (len == gs && (gs == 32 || gs == 64)) {
    // class maxima over vectors j = 0 .. gs/8-1, paired (0,1), (2,3), then
    // (01, 23), and (0123, 4567); then lanes i with i+4, 0 with 2 and 1 with 3, 0 with 1
    float m[8];
    for (int i = 0; i < 8; ++i) {
      auto a = [&](int j) { return __builtin_fabsf(value(8 * j + i)); };
      const float lo = vmax_x86(vmax_x86(a(0), a(1)), vmax_x86(a(2), a(3)));
      m[i] = gs == 64 ? vmax_x86(lo, vmax_x86(vmax_x86(a(4), a(5)), vmax_x86(a(6), a(7)))) : lo;
    }
    wmax = vmax_x86(vmax_x86(vmax_x86(m[0], m[4]), vmax_x86(m[2], m[6])),
                    vmax_x86(vmax_x86(m[1], m[5]), vmax_x86(m[3], m[7])));
  } else {
    for (int i = 0; i < len; ++i) wmax = vmax_x86(__builtin_fabsf(value(i)), wmax);
  }
  float scale, recip;
  q8_scale(q8_floor(wmax), scale, recip);
  out_s[r * spr + g] = scale;
  for (int i = 0; i < len; ++i) out_q[start + i] = (int8_t)q8_code_byte_full(value(i) * recip);
}

template <int GS>
static void launch_flat(int8_t *out_q, float *out_s, const float *x, const float *gate, const float *up, long long n,
                        hipStream_t stream) {
  const long long n4 = n / 4;
  const dim3 grid(stream_blocks(n4));
  if (gate)
    enqueue((quantize_q8_flat_kernel<GS, true>), grid, dim3(kStreamBlock), 0, stream, out_q, out_s, x, gate,
                       up, n4);
  else
    enqueue((quantize_q8_flat_kernel<GS, false>), grid, dim3(kStreamBlock), 0, stream, out_q, out_s, x,
                       gate, up, n4);
}

static bool aligned(const void *p, size_t a) { return p == nullptr || ((uintptr_t)p % a) == 0; }

void launch_quantize_q8(int8_t *out_q, float *out_s, const float *x, const float *gate, const float *up, int rows,
                        int row_len, int gs, hipStream_t stream) {
  const long long n = (long long)rows * row_len;
  const bool flat = (gs == 32 || gs == 64) && row_len % gs == 0 && aligned(out_q, 4) && aligned(x, 16) &&
                    aligned(gate, 16) && aligned(up, 16);
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
    enqueue((quantize_q8_generic_kernel<true>), dim3(blocks), dim3(256), 0, stream, out_q, out_s, x, gate,
                       up, rows, row_len, gs);
  else
    enqueue((quantize_q8_generic_kernel<false>), dim3(blocks), dim3(256), 0, stream, out_q, out_s, x, gate,
                       up, rows, row_len, gs);
}

}  // namespace v7g
