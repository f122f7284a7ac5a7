// k_rmsnorm_rope.hip -- per-head RMSNorm + rotate-half RoPE over Q/K heads, gfx950.
//
// Reference: v7s_rmsnorm_rope_heads(buf, n_heads, head_dim, norm_weight, cos,
// sin, pos, rope_max_dim), src/asm/rmsnorm_rope_dispatch.inc:11-52, one job per
// head running RMSNORM_ROPE_BODY (src/asm/v7_macros.inc:263-340):
//   sumsq: 32-element blocks, elements 0-7 of each block into accumulator A,
//          8-15 into B, 16-23 into C, 24-31 into D (FMA); (A+B)+(C+D); HADD_YMM.
//   scale: 1/sqrt(sumsq/head_dim + eps).
//   pos == 0: x = (x*scale)*w, no rotation.
//   pos  > 0: xe = (x_j*scale)*w_j, xo = (x_{j+h}*scale)*w_{j+h},
//             out_j = fma(-xo, sin_j, xe*cos_j), out_{j+h} = fma(xo, cos_j, xe*sin_j).
// cos/sin rows are table + pos*rope_max_dim.
// The same kernels run the whole Q/K/V stage of a prefill token (src/asm/
// prefill_q8.inc:848-883) in one pass: per side an optional QKV bias add
// first (PQ_BIAS_ADD, src/asm/v7_macros.inc:366-383), then RMSNorm+RoPE, or
// RoPE only when the side has no norm weight (v7s_rope_only_heads,
// src/asm/rope_only_kernel.inc:11-53: the rotation above applied to x
// itself), nothing more for V; then the f32 head in place and/or its binary16
// KV-cache row (v7s_kv_pack_f16, src/asm/kv_f16c.inc).
//
// gfx950 layout: 8 lanes per head.  Lane m of a head holds the float4 at
// x[4m + 32k] for every 32-element block k, so each of the 32 FMA chains (YMM
// accumulator q, lane j <-> element 8q + j of every block) is lane-local and
// runs in the reference order; the xor exchanges 2, 4, 1 are exactly the
// (A+B)+(C+D) and HADD_YMM pairings.  When head_dim % 64 == 0 the rotate-half
// partner of block k is block k + K/2 in the same lane, so the rotation
// happens in registers; otherwise it is in lane m ^ 4 (the wave kernel's
// lane exchange) or goes through LDS (the per-lane kernel).  At head_dim 256
// a head spans 16 lanes, the two halves holding alternate blocks, and the
// chains pass from one half to the other after each block (same order).  A
// wave holds heads of one side of one token, or, where a side's head count
// does not fill whole waves and the call is large, (token, head) pairs of one
// side over a group of tokens (the flat layout).  Heads are read and written
// in place with streaming loads and stores (the norm weights and the cos/sin
// rows, shared by every head of a token, stay cached).  The result is
// bit-identical to the reference.
#include "v7g_device.h"
#include "v7g_internal.h"

namespace v7g {

struct RopeArgs {
  RopeSide side[3];
  int n_sides;
  int n_heads0, n_heads01;  // side 0 heads; sides 0 + 1 heads
  int heads_per_token;      // heads of all sides
  unsigned n_heads;         // n_tokens * heads_per_token
  unsigned n_tokens;
  // The wave kernels' grid: per token, ceil(heads / 8) waves for each side (heads / 4 at head_dim 256);
  // the flat layout's: per group of 8 tokens (4 at head_dim 256), heads waves for each side
  // (waves_per_token then counts a group).
  int wave0, wave01;        // side 0 waves; sides 0 + 1 waves
  int waves_per_token;
  unsigned n_waves;         // n_tokens * waves_per_token
  int head_dim;
  const float *cos_table;
  const float *sin_table;
  const int32_t *positions;  // nullptr: pos = pos0 + token
  int pos0;
  int rope_max_dim;
  int table_rows;  // positions available in cos/sin; others give NaN rows
  float eps;
};

// The fields a wave reads before its first load (its wave index fields,
// the token count, the positions and the tables) also travel ahead of the
// argument block as scalar kernel arguments (14 dwords): the firmware
// preloads the first 14 argument dwords into SGPRs at wave launch, where a
// field of the by-value block is fetched with a scalar load and waited for
// (about 0.4 us of every launch at 32 + 8 heads of 128, from 1024 to 16384
// tokens).  The kernel rebuilds the block with them (RopeArgs a =
// V7G_ROPE_ARGS); enqueue_rope passes them.
#define V7G_ROPE_HOT                                                                                             \
  unsigned hot_n_waves, int hot_waves_per_token, int hot_wave0, int hot_wave01, const int32_t *hot_positions, \
      const float *hot_cos, const float *hot_sin, int hot_rope_max_dim, int hot_table_rows, int hot_pos0,    \
      unsigned hot_n_tokens, RopeArgs a_in
#define V7G_ROPE_ARGS                                                                                        \
  with_hot(a_in, hot_n_waves, hot_waves_per_token, hot_wave0, hot_wave01, hot_positions, hot_cos, hot_sin, \
           hot_rope_max_dim, hot_table_rows, hot_pos0, hot_n_tokens)

__device__ __forceinline__ RopeArgs with_hot(RopeArgs a, unsigned n_waves, int waves_per_token, int wave0, int wave01,
                                             const int32_t *positions, const float *cos_table,
                                             const float *sin_table, int rope_max_dim, int table_rows, int pos0,
                                             unsigned n_tokens) {
  a.n_waves = n_waves;
  a.waves_per_token = waves_per_token;
  a.wave0 = wave0;
  a.wave01 = wave01;
  a.positions = positions;
  a.cos_table = cos_table;
  a.sin_table = sin_table;
  a.rope_max_dim = rope_max_dim;
  a.table_rows = table_rows;
  a.pos0 = pos0;
  a.n_tokens = n_tokens;
  return a;
}

template <typename... KArgs>
static void enqueue_rope(void (*kernel)(KArgs...), dim3 grid, hipStream_t stream, const RopeArgs &a) {
  enqueue(kernel, grid, dim3(256), 0, stream, a.n_waves, a.waves_per_token, a.wave0, a.wave01, a.positions,
          a.cos_table, a.sin_table, a.rope_max_dim, a.table_rows, a.pos0, a.n_tokens, a);
}

// Where head f (flat over tokens x heads of all sides) lives, and what to do with it.
struct HeadRef {
  float *x;        // this lane's first float of the head
  const float *w;  // norm weight (lane offset) or nullptr: no RMSNorm
  const float *b;  // bias (lane offset) or nullptr
  uint16_t *kc;    // binary16 cache address (lane offset) or nullptr
  int pos;
  bool live;
  bool bad_pos;
  bool rotate;
  bool write_f32;
};

__device__ __forceinline__ HeadRef head_ref(const RopeArgs &a, unsigned f, int m) {
  HeadRef r;
  r.live = f < a.n_heads;
  const unsigned ff = r.live ? f : 0u;
  const unsigned t = ff / (unsigned)a.heads_per_token;
  const int h = (int)(ff - t * (unsigned)a.heads_per_token);
  const int sd = h < a.n_heads0 ? 0 : (h < a.n_heads01 ? 1 : 2);
  const int hs = h - (sd == 0 ? 0 : (sd == 1 ? a.n_heads0 : a.n_heads01));
  const RopeSide &S = a.side[sd];
  const size_t in_head = (size_t)hs * a.head_dim + 4 * m;
  r.x = S.buf + (size_t)t * (size_t)S.token_stride + in_head;
  r.w = S.norm_weight ? S.norm_weight + 4 * m : nullptr;
  r.b = S.bias ? S.bias + in_head : nullptr;
  r.kc = S.cache ? S.cache + (size_t)t * (size_t)S.cache_stride + in_head : nullptr;
  r.rotate = S.rotate;
  r.write_f32 = !S.cache || S.keep_f32;
  int pos = a.positions ? a.positions[t] : a.pos0 + (int)t;
  // A position outside the tables cannot be read: its rotated heads become NaN.
  r.bad_pos = S.rotate && pos != 0 && (unsigned)pos >= (unsigned)a.table_rows;
  r.pos = r.bad_pos ? 0 : pos;
  return r;
}

template <int K>
__device__ __forceinline__ float head_scale(const float4 (&x)[K], int head_dim, float eps) {
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    acc.x = __builtin_fmaf(x[k].x, x[k].x, acc.x);
    acc.y = __builtin_fmaf(x[k].y, x[k].y, acc.y);
    acc.z = __builtin_fmaf(x[k].z, x[k].z, acc.z);
    acc.w = __builtin_fmaf(x[k].w, x[k].w, acc.w);
  }
  // A+B and C+D: lane m with m^2; (A+B)+(C+D): m with m^4; HADD_YMM first
  // step v_i + v_{i+4}: m with m^1 (lanes 0/1 hold YMM lanes 0-3 / 4-7).
  acc.x = acc.x + xor_f(acc.x, 2); acc.y = acc.y + xor_f(acc.y, 2);
  acc.z = acc.z + xor_f(acc.z, 2); acc.w = acc.w + xor_f(acc.w, 2);
  acc.x = acc.x + xor_f(acc.x, 4); acc.y = acc.y + xor_f(acc.y, 4);
  acc.z = acc.z + xor_f(acc.z, 4); acc.w = acc.w + xor_f(acc.w, 4);
  acc.x = acc.x + xor_f(acc.x, 1); acc.y = acc.y + xor_f(acc.y, 1);
  acc.z = acc.z + xor_f(acc.z, 1); acc.w = acc.w + xor_f(acc.w, 1);
  const float t0 = acc.x + acc.y;
  const float t2 = acc.z + acc.w;
  return rms_scale(t0 + t2, (float)head_dim, eps);
}

// Loads the head (streaming) and adds the bias, as PQ_BIAS_ADD does before
// the norm: x = x + b.
template <int K>
__device__ __forceinline__ void load_head(float4 (&x)[K], const HeadRef &h) {
#pragma unroll
  for (int k = 0; k < K; ++k) {
    x[k] = h.live ? ld_stream4(h.x + 32 * k) : make_float4(0.f, 0.f, 0.f, 0.f);
    if (h.b) {
      const float4 b = *reinterpret_cast<const float4 *>(h.b + 32 * k);
      x[k] = make_float4(x[k].x + b.x, x[k].y + b.y, x[k].z + b.z, x[k].w + b.w);
    }
  }
}

// xn = (x * s) * w with the RMS scale of the head, or xn = x without a norm
// weight; NaN for a rotating head whose position is outside the tables.  The
// branch on h.w is uniform over the 8 lanes of a head, which are the only
// lanes the scale's exchanges read.
template <int K>
__device__ __forceinline__ void normalise(float4 (&xn)[K], const float4 (&x)[K], const HeadRef &h, int head_dim,
                                          float eps) {
  if (h.w) {
    const float s = head_scale<K>(x, head_dim, eps);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const float4 w = *reinterpret_cast<const float4 *>(h.w + 32 * k);
      xn[k] = make_float4((x[k].x * s) * w.x, (x[k].y * s) * w.y, (x[k].z * s) * w.z, (x[k].w * s) * w.w);
    }
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) xn[k] = x[k];
  }
  if (h.bad_pos) {
    const float q = __builtin_nanf("");
#pragma unroll
    for (int k = 0; k < K; ++k) xn[k] = make_float4(q, q, q, q);
  }
}

// The head's results: f32 in place, and/or binary16 into its cache row.
template <int K>
__device__ __forceinline__ void store_head(const HeadRef &h, const float4 (&xn)[K]) {
  if (h.write_f32) {
#pragma unroll
    for (int k = 0; k < K; ++k) st_stream4(h.x + 32 * k, xn[k]);
  }
  if (h.kc) {
#pragma unroll
    for (int k = 0; k < K; ++k) st_stream_u2(reinterpret_cast<uint32_t *>(h.kc + 32 * k), pack4_f16(xn[k]));
  }
}

// head_dim % 64 == 0: HPU heads per 8-lane unit, rotation in registers.  One
// head per unit measured fastest inside the per-layer chain (more heads per
// unit raise the registers per thread and lower occupancy).
template <int K, int HPU>
__global__ __launch_bounds__(256) void rmsnorm_rope_reg_kernel(RopeArgs a) {
  constexpr int KH = K / 2;
  const int m = threadIdx.x & 7;
  const unsigned unit = (blockIdx.x * 256u + threadIdx.x) >> 3;
  HeadRef hr[HPU];
  float4 x[HPU][K];
#pragma unroll
  for (int e = 0; e < HPU; ++e) {
    hr[e] = head_ref(a, unit * HPU + e, m);
    load_head<K>(x[e], hr[e]);
  }
#pragma unroll
  for (int e = 0; e < HPU; ++e) {
    float4 xn[K];
    normalise<K>(xn, x[e], hr[e], 32 * K, a.eps);
    if (hr[e].rotate && hr[e].pos != 0) {
      const size_t row = (size_t)hr[e].pos * (size_t)a.rope_max_dim + 4 * m;
      const float *cr = a.cos_table + row;
      const float *sr = a.sin_table + row;
#pragma unroll
      for (int k = 0; k < KH; ++k) {
        const float4 c = *reinterpret_cast<const float4 *>(cr + 32 * k);
        const float4 sn = *reinterpret_cast<const float4 *>(sr + 32 * k);
        const float4 ev = xn[k], od = xn[k + KH];
        xn[k] = make_float4(__builtin_fmaf(-od.x, sn.x, ev.x * c.x), __builtin_fmaf(-od.y, sn.y, ev.y * c.y),
                            __builtin_fmaf(-od.z, sn.z, ev.z * c.z), __builtin_fmaf(-od.w, sn.w, ev.w * c.w));
        xn[k + KH] = make_float4(__builtin_fmaf(od.x, c.x, ev.x * sn.x), __builtin_fmaf(od.y, c.y, ev.y * sn.y),
                                 __builtin_fmaf(od.z, c.z, ev.z * sn.z), __builtin_fmaf(od.w, c.w, ev.w * sn.w));
      }
    }
    if (hr[e].live) store_head<K>(hr[e], xn);
  }
}

// head_dim % 64 == 32: the partner of element e is e +- HD/2, in another lane;
// every head of the block (32 of them, HD floats each) goes through LDS.  All
// threads reach the barrier; the rotation itself is skipped at pos 0 and for
// sides that do not rotate.
template <int K>
__global__ __launch_bounds__(256) void rmsnorm_rope_lds_kernel(RopeArgs a) {
  constexpr int HD = 32 * K;
  constexpr int HALF = HD / 2;
  __shared__ __attribute__((aligned(16))) float lds[32 * HD];  // 16-byte LDS stores of the float4 chunks
  const int m = threadIdx.x & 7;
  const unsigned unit = (blockIdx.x * 256u + threadIdx.x) >> 3;
  const HeadRef hr = head_ref(a, unit, m);
  float4 x[K];
  load_head<K>(x, hr);
  float4 xn[K];
  normalise<K>(xn, x, hr, HD, a.eps);
  float *hb = lds + (threadIdx.x >> 3) * HD;
#pragma unroll
  for (int k = 0; k < K; ++k) *reinterpret_cast<float4 *>(hb + 4 * m + 32 * k) = xn[k];
  __syncthreads();
  if (hr.rotate && hr.pos != 0) {
    const size_t row = (size_t)hr.pos * (size_t)a.rope_max_dim;
    const float *cr = a.cos_table + row;
    const float *sr = a.sin_table + row;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const float cur[4] = {xn[k].x, xn[k].y, xn[k].z, xn[k].w};
      float res[4];
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {
        const int e = 4 * m + 32 * k + c4;
        if (e < HALF) {
          res[c4] = __builtin_fmaf(-hb[e + HALF], sr[e], cur[c4] * cr[e]);
        } else {
          const int j = e - HALF;
          res[c4] = __builtin_fmaf(cur[c4], cr[j], hb[j] * sr[j]);
        }
      }
      xn[k] = make_float4(res[0], res[1], res[2], res[3]);
    }
  }
  if (hr.live) store_head<K>(hr, xn);
}

// Zeros that stand in for a missing norm weight or cos/sin row, so that every
// lane issues the same loads (the results are not used).  K <= 8 reads at
// most float 4*7 + 32*7 + 3.
__device__ float kZeroRow[256] = {};  // never written; not const, so it stays in the global address space

// head_dim 64 to 224: each wave takes up to 8 heads of one side of one token
// (ceil(heads / 8) waves per side and token), so the side, its descriptor
// fields and the position are read once per wave with scalar loads, instead
// of per lane from the kernel arguments with vector loads, whose in-order
// completion made every lane wait for its head's data before it could even
// request the norm weights, and again before the cos/sin rows.  Here a lane's
// head, weight and cos/sin loads are all in flight together (a side without
// weights or rotation reads kZeroRow instead).  Lanes past the side's last
// head repeat that head's loads, which the same instructions fetch anyway, and
// store nothing.  The arithmetic is rmsnorm_rope_reg_kernel's.  At most 64
// VGPRs (8 waves per SIMD) up to head_dim 128; 86-127 from 160 to 224, where
// having every load in flight still beats the per-lane kernels' occupancy.
//
// head_dim % 64 == 32 (odd K): the rotate-half partner of lane m's block k is
// in lane m ^ 4 of the same head, in block k + J (k - J - 1) for lanes 0..3
// and k + J + 1 (k - J) for lanes 4..7 in the first (second) half, J = (K-1)/2;
// each lane sends the block its partner needs (a per-lane choice between two
// compile-time blocks) through one xor-4 exchange per block, and loads the
// cos/sin entries of its own elements (j = e in the first half, e - hd/2 in
// the second).
// BW (some side has a bias, and no side has both a bias and a norm weight:
// the QKV bias of a model without Q/K norms): a side's bias goes through the
// weight registers, with the other loads.  Otherwise a bias is read after the
// other loads, one load at a time, each waited for (the compiler's choice
// within 64 VGPRs), which cost the 28 Q / 4 KV head stage of 128 with QKV
// bias 5.5 points of the HBM peak before BW; without a bias that form of the
// kernel measured about 1 us faster on the Q/K/V stage than one with the bias
// code taken out.
template <int K, bool BW>
__global__ __launch_bounds__(256, (K == 2 || K == 3 || K == 4) ? 8 : 1) void rmsnorm_rope_wave_kernel(V7G_ROPE_HOT) {
  const RopeArgs a = V7G_ROPE_ARGS;
  static_assert(K >= 2 && K <= 7, "head_dim 64 to 224 (256: rmsnorm_rope_wave16_kernel)");
  constexpr bool ODD = K % 2 == 1;
  constexpr int KH = K / 2;         // even K: the partner of block k is block k + KH in the same lane
  constexpr int KC = ODD ? K : KH;  // cos/sin float4 per lane
  constexpr int J = (K - 1) / 2;
  const int m = threadIdx.x & 7;
  const bool lo = m < 4;
  const unsigned wi = __builtin_amdgcn_readfirstlane((blockIdx.x * 256u + threadIdx.x) >> 6);  // wave index
  const bool live_wave = wi < a.n_waves;
  const unsigned wvv = live_wave ? wi : 0u;
  const unsigned t = wvv / (unsigned)a.waves_per_token;
  const int r = (int)(wvv - t * (unsigned)a.waves_per_token);
  const int sd = r < a.wave0 ? 0 : (r < a.wave01 ? 1 : 2);
  const RopeSide S = a.side[sd];  // a copy: every field is requested before the barrier below
  const int hs_raw = 8 * (r - (sd == 0 ? 0 : (sd == 1 ? a.wave0 : a.wave01))) + ((threadIdx.x & 63) >> 3);
  const bool live = live_wave && hs_raw < S.n_heads;
  const int hs = hs_raw < S.n_heads ? hs_raw : S.n_heads - 1;
  const size_t in_head = (size_t)hs * (32 * K) + 4 * m;
  float *x = S.buf + (size_t)t * (size_t)S.token_stride + in_head;
  int pos = a.positions ? a.positions[t] : a.pos0 + (int)t;
  // The side's fields and the position are requested together, in one round
  // of scalar loads, before the head's loads are addressed.
  asm volatile("" ::: "memory");
  // A position outside the tables cannot be read: its rotated heads become NaN.
  const bool bad_pos = S.rotate && pos != 0 && (unsigned)pos >= (unsigned)a.table_rows;
  if (bad_pos) pos = 0;
  const bool rot = S.rotate && pos != 0;
  const size_t row = (size_t)pos * (size_t)a.rope_max_dim + 4 * m;
  // BW: a side's bias is read into the weight registers, through a
  // wave-uniform base and a 32-bit lane offset, so that the loads address
  // through a scalar base as the norm weight's do.
  const float *wp;
  bool bias_in_w = false;
  if constexpr (BW) {
    bias_in_w = S.bias != nullptr;
    const float *wbase = S.norm_weight ? S.norm_weight : (bias_in_w ? S.bias : kZeroRow);
    wp = wbase + (bias_in_w ? (unsigned)in_head : 4u * m);
  } else {
    wp = S.norm_weight ? S.norm_weight + 4 * m : kZeroRow + 4 * m;
  }
  const float *cp = rot ? a.cos_table + row : kZeroRow + 4 * m;
  const float *sp = rot ? a.sin_table + row : kZeroRow + 4 * m;
  // odd K: whether the lane's block k lies in the first half of the head
  auto first_half = [&](int k) { return lo ? k <= J : k < J; };
  float4 xv[K], wv[K], c[KC], sn[KC];
#pragma unroll
  for (int k = 0; k < K; ++k) xv[k] = ld_stream4(x + 32 * k);
#pragma unroll
  for (int k = 0; k < K; ++k) wv[k] = *reinterpret_cast<const float4 *>(wp + 32 * k);
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int off = (!ODD || first_half(k)) ? 32 * k : 32 * k - 16 * K;
    c[k] = *reinterpret_cast<const float4 *>(cp + off);
    sn[k] = *reinterpret_cast<const float4 *>(sp + off);
  }
  // The loads above are issued here, ahead of the branches below (the
  // compiler would otherwise sink the weight and table loads past them).
  asm volatile("" ::: "memory");
  if constexpr (BW) {
    if (bias_in_w) {
#pragma unroll
      for (int k = 0; k < K; ++k)
        xv[k] = make_float4(xv[k].x + wv[k].x, xv[k].y + wv[k].y, xv[k].z + wv[k].z, xv[k].w + wv[k].w);
    }
  } else if (S.bias) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const float4 b = *reinterpret_cast<const float4 *>(S.bias + in_head + 32 * k);
      xv[k] = make_float4(xv[k].x + b.x, xv[k].y + b.y, xv[k].z + b.z, xv[k].w + b.w);
    }
  }
  float4 xn[K];
  if (S.norm_weight) {
    const float s = head_scale<K>(xv, 32 * K, a.eps);
#pragma unroll
    for (int k = 0; k < K; ++k)
      xn[k] = make_float4((xv[k].x * s) * wv[k].x, (xv[k].y * s) * wv[k].y, (xv[k].z * s) * wv[k].z,
                          (xv[k].w * s) * wv[k].w);
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) xn[k] = xv[k];
  }
  if (bad_pos) {
    const float q = __builtin_nanf("");
#pragma unroll
    for (int k = 0; k < K; ++k) xn[k] = make_float4(q, q, q, q);
  }
  if (rot && !ODD) {
#pragma unroll
    for (int k = 0; k < KH; ++k) {
      const float4 ev = xn[k], od = xn[k + KH];
      xn[k] = make_float4(__builtin_fmaf(-od.x, sn[k].x, ev.x * c[k].x), __builtin_fmaf(-od.y, sn[k].y, ev.y * c[k].y),
                          __builtin_fmaf(-od.z, sn[k].z, ev.z * c[k].z), __builtin_fmaf(-od.w, sn[k].w, ev.w * c[k].w));
      xn[k + KH] = make_float4(__builtin_fmaf(od.x, c[k].x, ev.x * sn[k].x), __builtin_fmaf(od.y, c[k].y, ev.y * sn[k].y),
                               __builtin_fmaf(od.z, c[k].z, ev.z * sn[k].z), __builtin_fmaf(od.w, c[k].w, ev.w * sn[k].w));
    }
  }
  if (rot && ODD) {  // rot is uniform over the wave: every lane takes part in the exchanges
    float4 part[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      // the block this lane's partner (lane m ^ 4, in the other half of the 8 lanes) needs for its block k
      const int kp_for_lo = k <= J ? k + J : k - J - 1;      // partner in lanes 0..3
      const int kp_for_hi = k <= J - 1 ? k + J + 1 : k - J;  // partner in lanes 4..7
      const float4 snd = lo ? xn[kp_for_hi] : xn[kp_for_lo];
      part[k] = make_float4(xor_f(snd.x, 4), xor_f(snd.y, 4), xor_f(snd.z, 4), xor_f(snd.w, 4));
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const float4 me = xn[k], pa = part[k];
      if (first_half(k))  // me = x_j, partner = x_{j+h}
        xn[k] = make_float4(__builtin_fmaf(-pa.x, sn[k].x, me.x * c[k].x), __builtin_fmaf(-pa.y, sn[k].y, me.y * c[k].y),
                            __builtin_fmaf(-pa.z, sn[k].z, me.z * c[k].z), __builtin_fmaf(-pa.w, sn[k].w, me.w * c[k].w));
      else  // me = x_{j+h}, partner = x_j
        xn[k] = make_float4(__builtin_fmaf(me.x, c[k].x, pa.x * sn[k].x), __builtin_fmaf(me.y, c[k].y, pa.y * sn[k].y),
                            __builtin_fmaf(me.z, c[k].z, pa.z * sn[k].z), __builtin_fmaf(me.w, c[k].w, pa.w * sn[k].w));
    }
  }
  if (live) {
    if (!S.cache || S.keep_f32) {
#pragma unroll
      for (int k = 0; k < K; ++k) st_stream4(x + 32 * k, xn[k]);
    }
    if (S.cache) {
      uint16_t *kc = S.cache + (size_t)t * (size_t)S.cache_stride + in_head;
#pragma unroll
      for (int k = 0; k < K; ++k) st_stream_u2(reinterpret_cast<uint32_t *>(kc + 32 * k), pack4_f16(xn[k]));
    }
  }
}

// head_dim 256 in 16 lanes per head (4 heads per wave): in the 8-lane layout
// a lane holds 8 float4 of the head and 8 of the weights (110 VGPRs, 4 waves
// per SIMD).  Here the two 8-lane halves take alternate 32-element blocks:
// lane (h, m) holds x[64k + 32h + 4m .. +3], k < 4, i.e. blocks 2k + h.  The
// 32 FMA chains still run in the reference's order, block 0 to 7: after
// block b the accumulators live in half b & 1, and one DPP rotation by 8
// within the 16-lane row hands them to the other half for block b + 1.  The
// (A+B)+(C+D) + HADD_YMM exchanges (lanes m ^ 2, ^ 4, ^ 1) run inside each
// half; half 1 holds the result and rotates the scale back to half 0.  The
// rotate-half partner of block b is block b + 4, the same half, two
// registers on (k + 2), so the rotation stays in registers; the cos/sin
// entries of a lane's first-half elements are j = 64k + 32h + 4m .. +3, k < 2.
// Same side mapping, loads and stores as rmsnorm_rope_wave_kernel.
__device__ __forceinline__ float ror8_f(float v) {  // lane l gets lane l ^ 8 of its 16-lane row
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
}

// FLAT (head counts that are not multiples of 4, from 1024 tokens): tokens go
// in groups of 4 and each side's (token, head) pairs of a group are dealt out
// 4 to a wave in token-major order (side s: n_s waves per group), as the flat
// layout of the 8-lane kernel below; the position, the table rows, the
// out-of-table NaN and the rotation are then per 16-lane group.
template <bool BW, bool FLAT = false>
__global__ __launch_bounds__(256, 8) void rmsnorm_rope_wave16_kernel(V7G_ROPE_HOT) {
  const RopeArgs a = V7G_ROPE_ARGS;
  constexpr int HD = 256;
  const int m = threadIdx.x & 7;
  const int h = (threadIdx.x >> 3) & 1;
  const unsigned lane_off = 32u * h + 4u * m;  // the lane's first element of its head
  const unsigned wi = __builtin_amdgcn_readfirstlane((blockIdx.x * 256u + threadIdx.x) >> 6);  // wave index
  const bool live_wave = wi < a.n_waves;
  const unsigned wvv = live_wave ? wi : 0u;
  const unsigned grp = wvv / (unsigned)a.waves_per_token;  // the token, or with FLAT the group of 4 tokens
  const int r = (int)(wvv - grp * (unsigned)a.waves_per_token);
  const int sd = r < a.wave0 ? 0 : (r < a.wave01 ? 1 : 2);
  const RopeSide S = a.side[sd];  // a copy: every field is requested here, in one round
  asm volatile("" ::: "memory");
  const int hs_raw = 4 * (r - (sd == 0 ? 0 : (sd == 1 ? a.wave0 : a.wave01))) + ((threadIdx.x & 63) >> 4);
  bool live;
  int hs;
  unsigned t;
  if constexpr (FLAT) {  // hs_raw is the pair's index among the side's 4 * n_heads pairs of the group
    const unsigned n_tokens = a.n_tokens;
    const unsigned tl = (unsigned)hs_raw / (unsigned)S.n_heads;
    hs = hs_raw - (int)(tl * (unsigned)S.n_heads);
    const unsigned tg = 4u * grp + tl;
    live = live_wave && tg < n_tokens;
    t = tg < n_tokens ? tg : n_tokens - 1;
  } else {
    live = live_wave && hs_raw < S.n_heads;
    hs = hs_raw < S.n_heads ? hs_raw : S.n_heads - 1;
    t = grp;
  }
  int pos = a.positions ? a.positions[t] : a.pos0 + (int)t;
  if constexpr (FLAT) asm volatile("" ::: "memory");  // the position's load goes out ahead of the head's
  const size_t in_head = (size_t)hs * HD + lane_off;
  float *x = S.buf + (size_t)t * (size_t)S.token_stride + in_head;
  // A position outside the tables cannot be read: its rotated heads become NaN.
  const bool bad_pos = S.rotate && pos != 0 && (unsigned)pos >= (unsigned)a.table_rows;
  if (bad_pos) pos = 0;
  const bool rot = S.rotate && pos != 0;
  const size_t row = (size_t)pos * (size_t)a.rope_max_dim + lane_off;
  const float *wp;
  bool bias_in_w = false;
  if constexpr (BW) {
    bias_in_w = S.bias != nullptr;
    const float *wbase = S.norm_weight ? S.norm_weight : (bias_in_w ? S.bias : kZeroRow);
    wp = wbase + (bias_in_w ? (unsigned)in_head : lane_off);
  } else {
    wp = S.norm_weight ? S.norm_weight + lane_off : kZeroRow + lane_off;
  }
  // kZeroRow covers floats up to lane_off + 64*3 + 3 <= 255
  const float *cp = rot ? a.cos_table + row : kZeroRow + lane_off;
  const float *sp = rot ? a.sin_table + row : kZeroRow + lane_off;
  float4 xv[4], wv[4], c[2], sn[2];
#pragma unroll
  for (int k = 0; k < 4; ++k) xv[k] = ld_stream4(x + 64 * k);
#pragma unroll
  for (int k = 0; k < 4; ++k) wv[k] = *reinterpret_cast<const float4 *>(wp + 64 * k);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    c[k] = *reinterpret_cast<const float4 *>(cp + 64 * k);
    sn[k] = *reinterpret_cast<const float4 *>(sp + 64 * k);
  }
  asm volatile("" ::: "memory");
  if constexpr (BW) {
    if (bias_in_w) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        xv[k] = make_float4(xv[k].x + wv[k].x, xv[k].y + wv[k].y, xv[k].z + wv[k].z, xv[k].w + wv[k].w);
    }
  } else if (S.bias) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float4 b = *reinterpret_cast<const float4 *>(S.bias + in_head + 64 * k);
      xv[k] = make_float4(xv[k].x + b.x, xv[k].y + b.y, xv[k].z + b.z, xv[k].w + b.w);
    }
  }
  float4 xn[4];
  if (S.norm_weight) {  // uniform over the wave: every lane takes part in the rotations
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      if (b > 0) acc = make_float4(ror8_f(acc.x), ror8_f(acc.y), ror8_f(acc.z), ror8_f(acc.w));
      const float4 v = xv[b >> 1];  // block b in half b & 1 (the other half's result is not used)
      acc = make_float4(__builtin_fmaf(v.x, v.x, acc.x), __builtin_fmaf(v.y, v.y, acc.y),
                        __builtin_fmaf(v.z, v.z, acc.z), __builtin_fmaf(v.w, v.w, acc.w));
    }
    acc.x = acc.x + xor_f(acc.x, 2); acc.y = acc.y + xor_f(acc.y, 2);
    acc.z = acc.z + xor_f(acc.z, 2); acc.w = acc.w + xor_f(acc.w, 2);
    acc.x = acc.x + xor_f(acc.x, 4); acc.y = acc.y + xor_f(acc.y, 4);
    acc.z = acc.z + xor_f(acc.z, 4); acc.w = acc.w + xor_f(acc.w, 4);
    acc.x = acc.x + xor_f(acc.x, 1); acc.y = acc.y + xor_f(acc.y, 1);
    acc.z = acc.z + xor_f(acc.z, 1); acc.w = acc.w + xor_f(acc.w, 1);
    const float t0 = acc.x + acc.y;
    const float t2 = acc.z + acc.w;
    const float s1 = rms_scale(t0 + t2, (float)HD, a.eps);  // valid in half 1
    const float s0 = ror8_f(s1);
    const float s = h ? s1 : s0;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      xn[k] = make_float4((xv[k].x * s) * wv[k].x, (xv[k].y * s) * wv[k].y, (xv[k].z * s) * wv[k].z,
                          (xv[k].w * s) * wv[k].w);
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) xn[k] = xv[k];
  }
  if (bad_pos) {
    const float q = __builtin_nanf("");
#pragma unroll
    for (int k = 0; k < 4; ++k) xn[k] = make_float4(q, q, q, q);
  }
  if (rot) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const float4 ev = xn[k], od = xn[k + 2];
      xn[k] = make_float4(__builtin_fmaf(-od.x, sn[k].x, ev.x * c[k].x), __builtin_fmaf(-od.y, sn[k].y, ev.y * c[k].y),
                          __builtin_fmaf(-od.z, sn[k].z, ev.z * c[k].z), __builtin_fmaf(-od.w, sn[k].w, ev.w * c[k].w));
      xn[k + 2] = make_float4(__builtin_fmaf(od.x, c[k].x, ev.x * sn[k].x), __builtin_fmaf(od.y, c[k].y, ev.y * sn[k].y),
                              __builtin_fmaf(od.z, c[k].z, ev.z * sn[k].z), __builtin_fmaf(od.w, c[k].w, ev.w * sn[k].w));
    }
  }
  if (live) {
    if (!S.cache || S.keep_f32) {
#pragma unroll
      for (int k = 0; k < 4; ++k) st_stream4(x + 64 * k, xn[k]);
    }
    if (S.cache) {
      uint16_t *kc = S.cache + (size_t)t * (size_t)S.cache_stride + in_head;
#pragma unroll
      for (int k = 0; k < 4; ++k) st_stream_u2(reinterpret_cast<uint32_t *>(kc + 64 * k), pack4_f16(xn[k]));
    }
  }
}

// Head counts that are not multiples of 8 (2 KV heads, 12, 14 or 28 Q heads),
// from 1024 tokens: rmsnorm_rope_wave_kernel's last wave of such a side holds
// only its leftover heads, and its idle lanes still issue every instruction (a
// side of 2 heads fills a quarter of its wave).  Here tokens go in groups of
// 8 and each side's (token, head) pairs of a group are dealt out 8 to a wave
// in token-major order, so every wave is full: side s takes n_s waves per group, and lane
// group g of wave j holds pair 8j + g, i.e. token 8*group + (8j + g) / n_s,
// head (8j + g) % n_s.  The side's descriptor stays wave-uniform; the position
// is per lane (its load goes out first, so the wait for it covers no other
// load), and so are the table rows, the out-of-table NaN and the pos == 0
// case, which keeps the unrotated head by a select (the rotation is computed
// for every lane; a head's 8 lanes share one token).  Arithmetic, order and
// bias handling (BW) are rmsnorm_rope_wave_kernel's.
template <int K, bool BW>
__global__ __launch_bounds__(256, (K == 2 || K == 3 || K == 4) ? 8 : 1) void rmsnorm_rope_flat_kernel(V7G_ROPE_HOT) {
  const RopeArgs a = V7G_ROPE_ARGS;
  static_assert(K >= 2 && K <= 7, "head_dim 64 to 224");
  constexpr bool ODD = K % 2 == 1;
  constexpr int KH = K / 2;
  constexpr int KC = ODD ? K : KH;
  constexpr int J = (K - 1) / 2;
  const int m = threadIdx.x & 7;
  const bool lo = m < 4;
  const unsigned wi = __builtin_amdgcn_readfirstlane((blockIdx.x * 256u + threadIdx.x) >> 6);  // wave index
  const bool live_wave = wi < a.n_waves;
  const unsigned wvv = live_wave ? wi : 0u;
  const unsigned grp = wvv / (unsigned)a.waves_per_token;  // waves_per_token: waves per group of 8 tokens
  const int r = (int)(wvv - grp * (unsigned)a.waves_per_token);
  const int sd = r < a.wave0 ? 0 : (r < a.wave01 ? 1 : 2);
  const RopeSide S = a.side[sd];  // a copy: every field is requested here, in one round
  asm volatile("" ::: "memory");
  const unsigned n_tokens = a.n_tokens;
  const unsigned nh = (unsigned)S.n_heads;
  const unsigned pair = 8u * (unsigned)(r - (sd == 0 ? 0 : (sd == 1 ? a.wave0 : a.wave01))) +
                        ((threadIdx.x & 63u) >> 3);
  const unsigned tl = pair / nh;
  const int h = (int)(pair - tl * nh);
  const unsigned t = 8u * grp + tl;
  const bool live = live_wave && t < n_tokens;
  const unsigned tt = t < n_tokens ? t : n_tokens - 1;
  int pos = a.positions ? a.positions[tt] : a.pos0 + (int)tt;
  asm volatile("" ::: "memory");  // the position's load goes out ahead of the head's
  const size_t in_head = (size_t)h * (32 * K) + 4 * m;
  float *x = S.buf + (size_t)tt * (size_t)S.token_stride + in_head;
  const float *wp;
  bool bias_in_w = false;
  if constexpr (BW) {
    bias_in_w = S.bias != nullptr;
    const float *wbase = S.norm_weight ? S.norm_weight : (bias_in_w ? S.bias : kZeroRow);
    wp = wbase + (bias_in_w ? (unsigned)in_head : 4u * m);
  } else {
    wp = S.norm_weight ? S.norm_weight + 4 * m : kZeroRow + 4 * m;
  }
  auto first_half = [&](int k) { return lo ? k <= J : k < J; };
  float4 xv[K], wv[K], c[KC], sn[KC];
#pragma unroll
  for (int k = 0; k < K; ++k) xv[k] = ld_stream4(x + 32 * k);
#pragma unroll
  for (int k = 0; k < K; ++k) wv[k] = *reinterpret_cast<const float4 *>(wp + 32 * k);
  asm volatile("" ::: "memory");
  // A position outside the tables cannot be read: its rotated heads become NaN.
  const bool bad_pos = S.rotate && pos != 0 && (unsigned)pos >= (unsigned)a.table_rows;
  if (bad_pos) pos = 0;
  const bool rot = S.rotate && pos != 0;
  const size_t row = (size_t)pos * (size_t)a.rope_max_dim + 4 * m;
  const float *cp = rot ? a.cos_table + row : kZeroRow + 4 * m;
  const float *sp = rot ? a.sin_table + row : kZeroRow + 4 * m;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int off = (!ODD || first_half(k)) ? 32 * k : 32 * k - 16 * K;
    c[k] = *reinterpret_cast<const float4 *>(cp + off);
    sn[k] = *reinterpret_cast<const float4 *>(sp + off);
  }
  asm volatile("" ::: "memory");
  if constexpr (BW) {
    if (bias_in_w) {
#pragma unroll
      for (int k = 0; k < K; ++k)
        xv[k] = make_float4(xv[k].x + wv[k].x, xv[k].y + wv[k].y, xv[k].z + wv[k].z, xv[k].w + wv[k].w);
    }
  } else if (S.bias) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const float4 b = *reinterpret_cast<const float4 *>(S.bias + in_head + 32 * k);
      xv[k] = make_float4(xv[k].x + b.x, xv[k].y + b.y, xv[k].z + b.z, xv[k].w + b.w);
    }
  }
  float4 xn[K];
  if (S.norm_weight) {
    const float sc = head_scale<K>(xv, 32 * K, a.eps);
#pragma unroll
    for (int k = 0; k < K; ++k)
      xn[k] = make_float4((xv[k].x * sc) * wv[k].x, (xv[k].y * sc) * wv[k].y, (xv[k].z * sc) * wv[k].z,
                          (xv[k].w * sc) * wv[k].w);
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) xn[k] = xv[k];
  }
  if (bad_pos) {
    const float q = __builtin_nanf("");
#pragma unroll
    for (int k = 0; k < K; ++k) xn[k] = make_float4(q, q, q, q);
  }
  float4 xr[K];  // the rotated head; kept only where rot holds
  if constexpr (!ODD) {
#pragma unroll
    for (int k = 0; k < KH; ++k) {
      const float4 ev = xn[k], od = xn[k + KH];
      xr[k] = make_float4(__builtin_fmaf(-od.x, sn[k].x, ev.x * c[k].x), __builtin_fmaf(-od.y, sn[k].y, ev.y * c[k].y),
                          __builtin_fmaf(-od.z, sn[k].z, ev.z * c[k].z), __builtin_fmaf(-od.w, sn[k].w, ev.w * c[k].w));
      xr[k + KH] = make_float4(__builtin_fmaf(od.x, c[k].x, ev.x * sn[k].x), __builtin_fmaf(od.y, c[k].y, ev.y * sn[k].y),
                               __builtin_fmaf(od.z, c[k].z, ev.z * sn[k].z), __builtin_fmaf(od.w, c[k].w, ev.w * sn[k].w));
    }
  } else {  // every lane takes part in the exchanges (a head's 8 lanes share its token, hence rot)
    float4 part[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int kp_for_lo = k <= J ? k + J : k - J - 1;      // partner in lanes 0..3
      const int kp_for_hi = k <= J - 1 ? k + J + 1 : k - J;  // partner in lanes 4..7
      const float4 snd = lo ? xn[kp_for_hi] : xn[kp_for_lo];
      part[k] = make_float4(xor_f(snd.x, 4), xor_f(snd.y, 4), xor_f(snd.z, 4), xor_f(snd.w, 4));
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const float4 me = xn[k], pa = part[k];
      if (first_half(k))
        xr[k] = make_float4(__builtin_fmaf(-pa.x, sn[k].x, me.x * c[k].x), __builtin_fmaf(-pa.y, sn[k].y, me.y * c[k].y),
                            __builtin_fmaf(-pa.z, sn[k].z, me.z * c[k].z), __builtin_fmaf(-pa.w, sn[k].w, me.w * c[k].w));
      else
        xr[k] = make_float4(__builtin_fmaf(me.x, c[k].x, pa.x * sn[k].x), __builtin_fmaf(me.y, c[k].y, pa.y * sn[k].y),
                            __builtin_fmaf(me.z, c[k].z, pa.z * sn[k].z), __builtin_fmaf(me.w, c[k].w, pa.w * sn[k].w));
    }
  }
  if (rot) {
#pragma unroll
    for (int k = 0; k < K; ++k) xn[k] = xr[k];
  }
  if (live) {
    if (!S.cache || S.keep_f32) {
#pragma unroll
      for (int k = 0; k < K; ++k) st_stream4(x + 32 * k, xn[k]);
    }
    if (S.cache) {
      uint16_t *kc = S.cache + (size_t)tt * (size_t)S.cache_stride + in_head;
#pragma unroll
      for (int k = 0; k < K; ++k) st_stream_u2(reinterpret_cast<uint32_t *>(kc + 32 * k), pack4_f16(xn[k]));
    }
  }
}

template <int K>
static void launch_k(const RopeArgs &a, bool flat, hipStream_t stream) {
  if constexpr (K <= 7) {
    if (flat && a.n_waves < (1u << 26)) {  // the host's layout: waves per group of 8 tokens
      bool any_bias = false, norm_and_bias = false;
      for (int i = 0; i < a.n_sides; ++i) {
        any_bias = any_bias || a.side[i].bias;
        norm_and_bias = norm_and_bias || (a.side[i].bias && a.side[i].norm_weight);
      }
      const dim3 grid((a.n_waves + 3u) / 4u);
      if (any_bias && !norm_and_bias)
        enqueue_rope((rmsnorm_rope_flat_kernel<K, true>), grid, stream, a);
      else
        enqueue_rope((rmsnorm_rope_flat_kernel<K, false>), grid, stream, a);
      return;
    }
  }
  if constexpr (K <= 8) {
    // 64 threads per wave index in 32 bits: n_waves < 2^26 (the general kernel covers the rest)
    if (a.n_waves < (1u << 26)) {
      bool any_bias = false, norm_and_bias = false;
      for (int i = 0; i < a.n_sides; ++i) {
        any_bias = any_bias || a.side[i].bias;
        norm_and_bias = norm_and_bias || (a.side[i].bias && a.side[i].norm_weight);
      }
      const bool bw = any_bias && !norm_and_bias;
      const dim3 grid((a.n_waves + 3u) / 4u);
      if constexpr (K == 8) {  // head_dim 256: 4 heads per wave (the host's wave layout)
        if (flat)
          bw ? enqueue_rope((rmsnorm_rope_wave16_kernel<true, true>), grid, stream, a)
             : enqueue_rope((rmsnorm_rope_wave16_kernel<false, true>), grid, stream, a);
        else if (bw)
          enqueue_rope((rmsnorm_rope_wave16_kernel<true>), grid, stream, a);
        else
          enqueue_rope((rmsnorm_rope_wave16_kernel<false>), grid, stream, a);
      } else if (bw) {
        enqueue_rope((rmsnorm_rope_wave_kernel<K, true>), grid, stream, a);
      } else {
        enqueue_rope((rmsnorm_rope_wave_kernel<K, false>), grid, stream, a);
      }
      return;
    }
  }
  if ((32 * K) % 64 == 0) {
    constexpr int HPU = 1;
    const unsigned units = (a.n_heads + HPU - 1) / HPU;
    enqueue((rmsnorm_rope_reg_kernel<K, HPU>), dim3((units + 31u) / 32u), dim3(256), 0, stream, a);
  } else {
    enqueue((rmsnorm_rope_lds_kernel<K>), dim3((a.n_heads + 31u) / 32u), dim3(256), 0, stream, a);
  }
}

void launch_rmsnorm_rope(const RopeSide *sides, int n_sides, int n_tokens, int head_dim, const float *cos_table,
                         const float *sin_table, const int32_t *positions, int pos0, int rope_max_dim, int table_rows,
                         float eps, hipStream_t stream) {
  RopeArgs a;
  a.n_sides = n_sides;
  for (int i = 0; i < 3; ++i) a.side[i] = sides[i < n_sides ? i : 0];
  a.n_heads0 = sides[0].n_heads;
  a.n_heads01 = a.n_heads0 + (n_sides > 1 ? sides[1].n_heads : 0);
  a.heads_per_token = a.n_heads01 + (n_sides > 2 ? sides[2].n_heads : 0);
  a.n_heads = (unsigned)n_tokens * (unsigned)a.heads_per_token;
  a.n_tokens = (unsigned)n_tokens;
  // heads per wave: 8 (8 lanes per head), 4 at head_dim 256 (16 lanes per head).  Where a side's
  // head count is not a multiple of that (up to head_dim 256), a large call takes the flat layout:
  // per group of 8 (4) tokens, n_heads waves for each side.  Its waves are full, but each lane
  // group waits for its own position and the grid has fewer waves, which costs more than the idle
  // lanes below 1024 tokens (2048 unless half the lanes of the per-token layout would idle).
  const int hpw = head_dim == 256 ? 4 : 8;
  int slots = 0;
  for (int i = 0; i < n_sides; ++i) slots += (sides[i].n_heads + hpw - 1) / hpw * hpw;
  const bool flat = head_dim <= 256 && slots != a.heads_per_token &&
                    (n_tokens >= 2048 || (n_tokens >= 1024 && 2 * a.heads_per_token <= slots));
  auto waves = [&](int i) {
    if (i >= n_sides) return 0;
    return flat ? sides[i].n_heads : (sides[i].n_heads + hpw - 1) / hpw;
  };
  a.wave0 = waves(0);
  a.wave01 = a.wave0 + waves(1);
  a.waves_per_token = a.wave01 + waves(2);
  const unsigned long long units =
      flat ? ((unsigned long long)n_tokens + hpw - 1) / hpw : (unsigned long long)n_tokens;
  const unsigned long long n_waves = units * (unsigned long long)a.waves_per_token;
  a.n_waves = n_waves < (1ull << 26) ? (unsigned)n_waves : (1u << 26);  // beyond: the general kernel
  a.head_dim = head_dim;
  a.cos_table = cos_table;
  a.sin_table = sin_table;
  a.positions = positions;
  a.pos0 = pos0;
  a.rope_max_dim = rope_max_dim;
  a.table_rows = table_rows;
  a.eps = eps;
  switch (head_dim / 32) {
    case 2: launch_k<2>(a, flat, stream); break;
    case 3: launch_k<3>(a, flat, stream); break;
    case 4: launch_k<4>(a, flat, stream); break;
    case 5: launch_k<5>(a, flat, stream); break;
    case 6: launch_k<6>(a, flat, stream); break;
    case 7: launch_k<7>(a, flat, stream); break;
    case 8: launch_k<8>(a, flat, stream); break;
    case 9: launch_k<9>(a, flat, stream); break;
    case 10: launch_k<10>(a, flat, stream); break;
    case 11: launch_k<11>(a, flat, stream); break;
    case 12: launch_k<12>(a, flat, stream); break;
    case 13: launch_k<13>(a, flat, stream); break;
    case 14: launch_k<14>(a, flat, stream); break;
    case 15: launch_k<15>(a, flat, stream); break;
    case 16: launch_k<16>(a, flat, stream); break;
    default: break;
  }
}

}  // namespace v7g
