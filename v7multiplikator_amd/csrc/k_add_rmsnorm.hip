// k_add_rmsnorm.hip -- fused residual-add + RMSNorm for gfx950.
//
// Reference: v7s_fused_add_rmsnorm(o, residual, add, weight, dim),
// src/asm/add_rmsnorm_kernel.inc:15-129.
//   Pass 1: residual = residual + add (stored in place); the sum of squares is
//           accumulated in four 8-lane YMM accumulators A..D by FMA.  Blocks of
//           8 floats that do not fill a 4-way group (blocks % 4) go first, all
//           into A; then each group of 4 blocks feeds A, B, C, D.
//   Reduce: (A+B)+(C+D) lane-wise, then HADD_YMM (v7_macros.inc:38-45).
//   Scale:  1/sqrt(sumsq/dim + eps), four IEEE operations.
//   Pass 2: o = (scale * residual) * weight.
// This kernel reproduces that order exactly, so its output is bit-identical.
// One workgroup per row: each thread keeps its float4 chunks of the row in
// registers (4*(tid + k*TPR) for k < KMAX), so pass 1 issues every load of
// residual and add together and pass 2 needs no second read; residual, add
// and o move as streaming loads and stores, the weight row stays cached.  The
// updated residual also goes to LDS, where 32 lanes of wave 0 replay the 32
// FMA chains (lane 8q + j is accumulator q, YMM lane j), conflict-free; the
// five-step xor exchange below is exactly the (A+B)+(C+D) + HADD_YMM pairing.
//
// The same row body serves the neighbours of this kernel in the reference:
//   v7s_rmsnorm (src/asm/rmsnorm_kernel.inc:12-75): no add, same order;
//   v7s_rmsnorm_quantize (src/asm/rmsnorm_quantize_kernel.inc:62-218): the
//     normalised row quantized per group of 64 exactly as v7d_quantize does;
//   and the Q8 decode step v7s_add_inplace -> v7s_rmsnorm_quantize
//     (src/asm/forward_q8.inc:386-387), fused here into one pass.
#include <type_traits>

#include "v7g_device.h"
#include "v7g_internal.h"

namespace v7g {

// The chain lane lam runs YMM accumulator q = v >> 3, lane j = v & 7 with
// v = chain_of_lane(lam), chosen so that lam = 8*q0 + 4*q1 + 2*j2 + j0 + 16*j1
// (q0, q1, j0..j2 the bits of q and j): the reduction's pairs are then lanes
// lam, lam+8 (A+B, C+D), lam, lam+4 ((A+B)+(C+D)), lam, lam+2 (v_i + v_{i+4}),
// lam, lam+1 (w0+w1, w2+w3) and lanes 0, 16 (the final sum).
__device__ __forceinline__ int chain_of_lane(int lam) {
  const int q = ((lam >> 3) & 1) | (((lam >> 2) & 1) << 1);
  const int j = (lam & 1) | (((lam >> 4) & 1) << 1) | (((lam >> 1) & 1) << 2);
  return 8 * q + j;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum of squares of a row of dim floats (dim % 32 == 0) staged at the padded
// layout, in the reference's order; called by a whole wave, returns the same
// value in every lane.  U: chain elements per register set (2U VGPRs).
template <int U>
__device__ __forceinline__ float padded_row_sumsq(const float *row, int dim) {
  const int lane = __lane_id();
  float acc = 0.0f;
  if (lane < 32) {
    const int v = chain_of_lane(lane);
    // element 32g + v sits at float 40g + v + 4*(v >> 4)
    const float *p = row + v + 4 * (v >> 4);
    const int steps = dim >> 5;
    if (steps % (2 * U) == 0) {
      // Two register sets of U chain elements: the LDS reads of one set are
      // in flight while the FMAs consume the other, so the chain waits on
      // LDS once instead of once per U steps.  Same FMAs, same order.  The
      // empty asm statements pass the accumulator through a point after each
      // set of reads, so the compiler neither sinks a read down to its use
      // nor hoists the FMAs above the reads of the other set.
      float a[U], b[U];
#pragma unroll
      for (int u = 0; u < U; ++u) a[u] = p[40 * u];
      int g0 = 0;
      for (; g0 + 2 * U < steps; g0 += 2 * U) {
#pragma unroll
        for (int u = 0; u < U; ++u) b[u] = p[40 * (g0 + U + u)];
        asm volatile("" : "+v"(acc)::"memory");
#pragma unroll
        for (int u = 0; u < U; ++u) acc = __builtin_fmaf(a[u], a[u], acc);
#pragma unroll
        for (int u = 0; u < U; ++u) a[u] = p[40 * (g0 + 2 * U + u)];
        asm volatile("" : "+v"(acc)::"memory");
#pragma unroll
        for (int u = 0; u < U; ++u) acc = __builtin_fmaf(b[u], b[u], acc);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) b[u] = p[40 * (g0 + U + u)];
      asm volatile("" : "+v"(acc)::"memory");
#pragma unroll
      for (int u = 0; u < U; ++u) acc = __builtin_fmaf(a[u], a[u], acc);
#pragma unroll
      for (int u = 0; u < U; ++u) acc = __builtin_fmaf(b[u], b[u], acc);
    } else {
#pragma unroll 16
      for (int g = 0; g < steps; ++g) {
        const float e = p[40 * g];
        acc = __builtin_fmaf(e, e, acc);
      }
    }
  }
  acc = acc + dpp_f<0x108>(acc);  // row_shl:8   A+B, C+D
  acc = acc + dpp_f<0x104>(acc);  // row_shl:4   (A+B)+(C+D)
  acc = acc + dpp_f<0x102>(acc);  // row_shl:2   HADD_YMM: v_i + v_{i+4}
  acc = acc + dpp_f<0x101>(acc);  // row_shl:1   w0+w1, w2+w3
  const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 0));
  const float hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 16));
  return lo + hi;
}

// A workgroup barrier for LDS only: unlike __syncthreads() it does not wait
// for the wave's global loads and stores (s_waitcnt lgkmcnt(0), not vmcnt).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ int padded(int m) { return 4 * (m + (m >> 2)); }

// One row.  ADD: the input is residual + add (residual updated in place),
// else x.  QGS == 0: o = (s*x)*w; QGS = 32 or 64: the normalised row is
// quantized in groups of QGS (codes q, scales q_s) and o is not written.
// o may alias residual (the row then ends as o, as in the reference).
// PAD (dim % 32 == 0, dim <= 12288): the row is staged at the padded layout and
// the chains' reduction runs as DPP row shifts (padded_row_sumsq); otherwise
// at the natural layout with the lane-exchange reduction, which also covers
// the leftover 8-float blocks of dim % 32 != 0.
// FIX (with PAD, dim == 4*TPR*KMAX): every chunk is live, so the loads and
// stores carry no bounds branches (whose merges cost waits on the outstanding
// loads); the fused-add form then also requests its weights right after the
// row's loads, ahead of the residual's stores, since vector memory operations
// retire in issue order and a weight load issued after those stores would
// wait for them (KMAX <= 4: with more chunks the weights would not fit in 64
// VGPRs beside the row).  TPR == 0 (FIX only): the thread count is the
// launch's blockDim.x and dim = 4*blockDim.x*KMAX; a compile-time TPR folds
// the chunk offsets into the instructions and measured about 2% faster.
template <int TPR, int KMAX, bool ADD, int QGS, bool PAD, bool FIX = false>
__device__ __forceinline__ void rms_row(float *o, int8_t *q, float *q_s, float *xin, const float *add,
                                        const float *weight, int dim, float eps) {
  static_assert(!FIX || PAD, "the fixed-length row uses the padded layout");
  static_assert(TPR > 0 || (FIX && QGS == 0), "a run-time thread count only for the fixed-length row");
  constexpr bool EARLY_W = FIX && ADD && QGS == 0 && KMAX <= 4;
  const int tpr = TPR ? TPR : (int)blockDim.x;
  if constexpr (FIX) dim = 4 * tpr * KMAX;
  extern __shared__ __attribute__((aligned(16))) float row[];
  const int tid = threadIdx.x;
  const size_t r = blockIdx.x;
  float *xr = xin + r * (size_t)dim;

  // Pass 1: load the row (and add), stage it in LDS.
  float4 x[KMAX], b[KMAX], w_early[EARLY_W ? KMAX : 1];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int i = 4 * (tid + k * tpr);
    if (FIX || i < dim) {
      x[k] = ld_stream4(xr + i);
      if constexpr (ADD) b[k] = ld_stream4(add + r * (size_t)dim + i);
    }
  }
  if constexpr (EARLY_W) {
#pragma unroll
    for (int k = 0; k < KMAX; ++k) w_early[k] = *reinterpret_cast<const float4 *>(weight + 4 * (tid + k * tpr));
  }
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int i = 4 * (tid + k * tpr);
    if (FIX || i < dim) {
      if constexpr (ADD) {
        x[k] = make_float4(x[k].x + b[k].x, x[k].y + b[k].y, x[k].z + b[k].z, x[k].w + b[k].w);
        st_stream4(xr + i, x[k]);
      }
      *reinterpret_cast<float4 *>(row + (PAD ? padded(tid + k * tpr) : i)) = x[k];
    }
  }
  __syncthreads();

  if constexpr (PAD) {
    // floats 16..19 of the padded layout are padding: the scale goes there
    if (tid < 64) {
      const float s0 = rms_scale(padded_row_sumsq<8>(row, dim), (float)dim, eps);
      if (tid == 0) row[16] = s0;
    }
  } else if (tid < 64) {
    // The 32 FMA chains: lane v = 8q + j is YMM accumulator q (A..D), lane j.
    float acc = 0.0f;
    if (tid < 32) {
      const int qa = tid >> 3, j = tid & 7;
      const int blocks = dim >> 3, left = blocks & 3, groups = blocks >> 2;
      if (qa == 0)
        for (int bb = 0; bb < left; ++bb) {
          const float v = row[8 * bb + j];
          acc = __builtin_fmaf(v, v, acc);
        }
      const float *p = row + 8 * (left + qa) + j;
#pragma unroll 16
      for (int g = 0; g < groups; ++g) {
        const float v = p[32 * g];
        acc = __builtin_fmaf(v, v, acc);
      }
    }
    // (A+B), (C+D): xor 8; then their sum: xor 16; HADD_YMM: xor 4, xor 1, xor 2.
    acc = acc + xor_f(acc, 8);
    acc = acc + xor_f(acc, 16);
    acc = acc + xor_f(acc, 4);
    acc = acc + xor_f(acc, 1);
    acc = acc + xor_f(acc, 2);
    // row[0] is dead now: only lane 0 read it (its first chain element), and
    // lane 0 is the writer; the other waves wait at the barrier below.
    if (tid == 0) row[0] = rms_scale(acc, (float)dim, eps);
  }
  __syncthreads();
  const float s = row[PAD ? 16 : 0];

  // Pass 2: n = (s * x) * w, then either stored or quantized.
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int i = 4 * (tid + k * tpr);
    const bool live = FIX || i < dim;
    float4 n = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) {
      float4 w;
      if constexpr (EARLY_W)
        w = w_early[k];
      else
        w = *reinterpret_cast<const float4 *>(weight + i);
      n = make_float4((s * x[k].x) * w.x, (s * x[k].y) * w.y, (s * x[k].z) * w.z, (s * x[k].w) * w.w);
    }
    if constexpr (QGS == 0) {
      if (live) st_stream4(o + r * (size_t)dim + i, n);
    } else {
      // QGS/4 consecutive lanes hold one group (dim % QGS == 0 and TPR % 16 == 0:
      // a group is entirely live or entirely past the row); every lane takes
      // part in the DPP butterfly, or, in a wave holding a NaN or an Inf, in
      // the reference's ordered vmaxps tree (rmsnorm_quantize_kernel.inc:158-186).
      constexpr int LPG = QGS / 4;
      float m = lane_absmax4(n);
      float scale, recip;
      uint32_t codes;
      if (!wave_any_nonfinite(m)) {
        m = (LPG == 8) ? group8_max(m) : group16_max(m);
        q8_scale_finite(m, scale, recip);
        codes = pack4_codes_finite(n, recip);
      } else {
        q8_scale(q8_floor(group_absmax_tree<QGS>(n)), scale, recip);
        codes = pack4_codes_full(n, recip);
      }
      if (live) {
        const size_t c = (r * (size_t)dim + i) >> 2;  // dword of 4 codes
        st_stream_u32(reinterpret_cast<uint32_t *>(q) + c, codes);
        if ((tid & (LPG - 1)) == 0) st_stream_f32(q_s + r * (size_t)(dim / QGS) + (i / QGS), scale);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// RMSNorm -> Q8 (and its fused-add form) for dim % 32 == 0, 512 <= dim <= 12288.
//
// One row per workgroup of dim/16 threads.  The row is read with coalesced
// dwordx4 loads (thread t: float4 chunks t + k*T, k < 4) and staged in LDS,
// chunk m at float 4*(m + m/4): 16 bytes of padding after every 64, so that
// the quantizer's reads below are free of bank conflicts.  Lanes 0..31 of
// wave 0 replay the reference's 32 FMA chains from LDS, then the exact
// (A+B)+(C+D) + HADD_YMM reduction runs as DPP row shifts (chain_of_lane
// places each partial sum where the shift finds its partner).  Each thread
// then quantizes 16 consecutive elements read back from LDS: the group max is
// a lane-local max and one or two quad DPP steps (4 or 2 lanes per group),
// the scale and reciprocal are computed once per 16 elements, and the 16
// codes leave as one 16-byte store.  The fused-add form writes the updated
// residual back with the loads' layout.  Same operations and order as
// rms_row, so the same bits; about 10% less time at [8192, 4096] than
// rms_row, whose 4-element-per-lane quantizer and lane-exchange reduction
// made the kernel issue-bound.  The LDS array is declared 16-byte aligned:
// with the element type's 4-byte alignment the compiler splits every float4
// access into two 8-byte ones.  The chains read their elements one register
// set ahead (16 elements; 8 in the fused-add form, which keeps the weights
// live across the chain and would otherwise exceed 64 VGPRs).

// TPB > 0: the block size, known at compile time (the common widths); 0: blockDim.x.
template <int TPB, int QGS, bool ADD>
__global__ __launch_bounds__(TPB ? TPB : 1024) void norm_q8_row16_kernel(int8_t *q, float *q_s, float *x,
                                                                         const float *add, const float *weight,
                                                                         int dim, float eps) {
  extern __shared__ __attribute__((aligned(16))) float row[];  // dim + dim/4 floats; floats 16..19 (padding) hold the scale
  const int t = threadIdx.x;
  const int T = TPB ? TPB : (int)blockDim.x;  // dim / 16
  if constexpr (TPB > 0) dim = 16 * TPB;
  const size_t r = blockIdx.x;
  float *xr = x + r * (size_t)dim;
  float4 w[4], v[4];
  // With the residual add, the weights are requested first: vector memory
  // counters retire in order, and a weight load issued after the residual's
  // stores would wait for them.  Without it they follow the staging.
  if constexpr (ADD) {
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = *reinterpret_cast<const float4 *>(weight + 16 * t + 4 * k);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = ld_stream4(xr + 4 * (t + k * T));
  if constexpr (ADD) {
    float4 b[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) b[k] = ld_stream4(add + r * (size_t)dim + 4 * (t + k * T));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[k] = make_float4(v[k].x + b[k].x, v[k].y + b[k].y, v[k].z + b[k].z, v[k].w + b[k].w);
      st_stream4(xr + 4 * (t + k * T), v[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) *reinterpret_cast<float4 *>(row + padded(t + k * T)) = v[k];
  lds_barrier();
  if (t < 64) {
    const float s0 = rms_scale(padded_row_sumsq<ADD ? 8 : 16>(row, dim), (float)dim, eps);
    if (t == 0) row[16] = s0;
  }
  if constexpr (!ADD) {
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = *reinterpret_cast<const float4 *>(weight + 16 * t + 4 * k);
  }
  lds_barrier();
  const float s = row[16];
  float n[16];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float4 xv = *reinterpret_cast<const float4 *>(row + 20 * t + 4 * k);  // chunks 4t .. 4t+3
    n[4 * k + 0] = (s * xv.x) * w[k].x;
    n[4 * k + 1] = (s * xv.y) * w[k].y;
    n[4 * k + 2] = (s * xv.z) * w[k].z;
    n[4 * k + 3] = (s * xv.w) * w[k].w;
  }
  // Group max: NaN-propagating lane max, then (no NaN or Inf in the wave) an
  // unsigned max over the group's 4 (GS 64) or 2 (GS 32) lanes, else the
  // reference's ordered vmaxps tree.
  float m = __builtin_elementwise_maximum(__builtin_fabsf(n[0]), __builtin_fabsf(n[1]));
#pragma unroll
  for (int i = 2; i < 16; ++i) m = __builtin_elementwise_maximum(m, __builtin_fabsf(n[i]));
  float scale, recip;
  uint32_t c[4];
  if (!wave_any_nonfinite(m)) {
    uint32_t u = __builtin_bit_cast(uint32_t, m);
    u = umax(u, dpp_u<DPP_QUAD_XOR1>(u));
    if constexpr (QGS == 64) u = umax(u, dpp_u<DPP_QUAD_XOR2>(u));
    q8_scale_finite(__builtin_bit_cast(float, u), scale, recip);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      c[k] = pack4_codes_finite(make_float4(n[4 * k], n[4 * k + 1], n[4 * k + 2], n[4 * k + 3]), recip);
  } else {
    q8_scale(q8_floor(group_absmax_tree16<QGS>(n)), scale, recip);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      c[k] = pack4_codes_full(make_float4(n[4 * k], n[4 * k + 1], n[4 * k + 2], n[4 * k + 3]), recip);
  }
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  const u4 cv = {c[0], c[1], c[2], c[3]};
  __builtin_nontemporal_store(cv, reinterpret_cast<u4 *>(q + r * (size_t)dim) + t);
  // every lane of the group stores the same scale to the same address (one store, no branch)
  st_stream_f32(q_s + r * (size_t)(dim / QGS) + t / (QGS / 16), scale);
}

template <int TPR, int KMAX, bool PAD, bool FIX>
__global__ __launch_bounds__(TPR ? TPR : 1024, (TPR == 0 && KMAX <= 4) ? 8 : 1) void fused_add_rmsnorm_kernel(float *o, float *residual, const float *add,
                                                                const float *weight, int dim, float eps) {
  rms_row<TPR, KMAX, true, 0, PAD, FIX>(o, nullptr, nullptr, residual, add, weight, dim, eps);
}

template <int TPR, int KMAX, bool PAD, bool FIX>
__global__ __launch_bounds__(TPR ? TPR : 1024, (TPR == 0 && KMAX <= 4) ? 8 : 1) void rmsnorm_kernel(float *o, float *x, const float *weight, int dim, float eps) {
  rms_row<TPR, KMAX, false, 0, PAD, FIX>(o, nullptr, nullptr, x, nullptr, weight, dim, eps);
}

template <int TPR, int KMAX, int QGS, bool PAD>
__global__ __launch_bounds__(TPR) void rmsnorm_quantize_kernel(int8_t *q, float *q_s, float *x, const float *weight,
                                                               int dim, float eps) {
  rms_row<TPR, KMAX, false, QGS, PAD>(nullptr, q, q_s, x, nullptr, weight, dim, eps);
}

template <int TPR, int KMAX, int QGS, bool PAD>
__global__ __launch_bounds__(TPR) void add_rmsnorm_quantize_kernel(int8_t *q, float *q_s, float *residual,
                                                                   const float *add, const float *weight, int dim,
                                                                   float eps) {
  rms_row<TPR, KMAX, true, QGS, PAD>(nullptr, q, q_s, residual, add, weight, dim, eps);
}

// Chooses threads per row and float4 chunks per thread for dim <= 16384
// (validated by the caller) and launches one workgroup per row.
struct RowLaunch {
  int rows, dim;
  hipStream_t stream;
  // the padded layout and DPP reduction: whole 32-float blocks, at most 64 KiB of LDS (5 bytes per element)
  bool pad() const { return dim % 32 == 0 && dim <= 12288; }
  // one float4 chunk per thread and k, all live: the fixed-length kernels
  bool fits(int tpr, int kmax) const { return pad() && dim == 4 * tpr * kmax; }
  size_t lds() const { return (size_t)(pad() ? dim + dim / 4 : dim) * sizeof(float); }
};

// Rows below 1024 floats take one wave each (up to 4 float4 chunks per lane)
// when there are more than 2048 of them: 256-thread rows would then need more
// than one round of the 8192 waves the GPU holds at once (256 CUs x 4 SIMDs x
// 8), one-wave rows fit 8192 rows in one ([4096, 384]: 7.4 -> 5.8 us; [8192,
// 896]: 21.9 -> 21.3 us).  Fewer rows keep the 256-thread row, whose loads
// spread over four waves (up to 0.6 us faster from 64 to 2048 rows).
template <template <int, int> class Op, typename... A>
static void dispatch_rows(const RowLaunch &L, A... args) {
  const bool wave_rows = L.rows > 2048;
  if (L.dim <= 256)
    Op<64, 1>::launch(L, args...);
  else if (L.dim <= 512 && wave_rows)
    Op<64, 2>::launch(L, args...);
  else if (L.dim <= 768 && wave_rows)
    Op<64, 3>::launch(L, args...);
  else if (L.dim < 1024 && wave_rows)
    Op<64, 4>::launch(L, args...);
  else if (L.dim <= 1024)
    Op<256, 1>::launch(L, args...);
  else if (L.dim <= 2048)
    Op<256, 2>::launch(L, args...);
  else if (L.dim <= 4096)
    Op<256, 4>::launch(L, args...);
  else if (L.dim <= 8192)
    Op<256, 8>::launch(L, args...);
  else
    Op<256, 16>::launch(L, args...);
}

template <int TPR, int KMAX>
struct AddNormOp {
  static void launch(const RowLaunch &L, float *o, float *residual, const float *add, const float *weight, float eps) {
    auto go = [&](auto kernel) {
      enqueue(kernel, dim3(L.rows), dim3(TPR), L.lds(), L.stream, o, residual, add, weight, L.dim, eps);
    };
    if (L.fits(TPR, KMAX))
      go(fused_add_rmsnorm_kernel<TPR, KMAX, true, true>);
    else if (L.pad())
      go(fused_add_rmsnorm_kernel<TPR, KMAX, true, false>);
    else
      go(fused_add_rmsnorm_kernel<TPR, KMAX, false, false>);
  }
};

template <int TPR, int KMAX>
struct NormOp {
  static void launch(const RowLaunch &L, float *o, float *x, const float *weight, float eps) {
    auto go = [&](auto kernel) { enqueue(kernel, dim3(L.rows), dim3(TPR), L.lds(), L.stream, o, x, weight, L.dim, eps); };
    if (L.fits(TPR, KMAX))
      go(rmsnorm_kernel<TPR, KMAX, true, true>);
    else if (L.pad())
      go(rmsnorm_kernel<TPR, KMAX, true, false>);
    else
      go(rmsnorm_kernel<TPR, KMAX, false, false>);
  }
};

template <int TPR, int KMAX>
struct NormQ8Op {
  static void launch(const RowLaunch &L, int8_t *q, float *q_s, float *x, const float *add, const float *weight,
                     float eps, int gs) {
    auto go_add = [&](auto kernel) {
      enqueue(kernel, dim3(L.rows), dim3(TPR), L.lds(), L.stream, q, q_s, x, add, weight, L.dim, eps);
    };
    auto go = [&](auto kernel) {
      enqueue(kernel, dim3(L.rows), dim3(TPR), L.lds(), L.stream, q, q_s, x, weight, L.dim, eps);
    };
    const bool pad = L.pad();
    if (add) {
      if (gs == 32)
        pad ? go_add(add_rmsnorm_quantize_kernel<TPR, KMAX, 32, true>)
            : go_add(add_rmsnorm_quantize_kernel<TPR, KMAX, 32, false>);
      else
        pad ? go_add(add_rmsnorm_quantize_kernel<TPR, KMAX, 64, true>)
            : go_add(add_rmsnorm_quantize_kernel<TPR, KMAX, 64, false>);
    } else {
      if (gs == 32)
        pad ? go(rmsnorm_quantize_kernel<TPR, KMAX, 32, true>) : go(rmsnorm_quantize_kernel<TPR, KMAX, 32, false>);
      else
        pad ? go(rmsnorm_quantize_kernel<TPR, KMAX, 64, true>) : go(rmsnorm_quantize_kernel<TPR, KMAX, 64, false>);
    }
  }
};

template <bool ADD, int TPR, int KMAX>
static auto fixed_row_kernel() {
  if constexpr (ADD)
    return fused_add_rmsnorm_kernel<TPR, KMAX, true, true>;
  else
    return rmsnorm_kernel<TPR, KMAX, true, true>;
}

// The fixed-length row at the widths between and above the powers of two,
// 1024 < dim <= 8192, dim % 256 == 0 (dim = 4 * threads * chunks): the shape
// that measured fastest at [8192, dim] for the common model widths, compiled
// in (2560, 3072, 3584, 3840, 5120, 8192: 1.5 to 2.5 points of the HBM peak
// above the general kernel, 8192 even); a run-time thread count with 2
// chunks per thread (1 where dim/4 is an odd multiple of 64) for the other
// multiples of 256 up to 4096 and of 512 up to 8192 (whole waves, at most
// 1024 threads).  2048 and 4096 keep the
// dispatch_rows shapes, which measured best.  Returns false where none applies.
template <bool ADD>
static bool launch_fixed_row(const RowLaunch &L, float *o, float *x, const float *add, const float *weight,
                             float eps) {
  if (L.dim <= 1024 || L.dim > 8192 || L.dim % 256 || L.dim == 2048 || L.dim == 4096) return false;
  auto go = [&](auto kernel, int tpr) {
    if constexpr (ADD)
      enqueue(kernel, dim3(L.rows), dim3(tpr), L.lds(), L.stream, o, x, add, weight, L.dim, eps);
    else
      enqueue(kernel, dim3(L.rows), dim3(tpr), L.lds(), L.stream, o, x, weight, L.dim, eps);
  };
  switch (L.dim) {
    case 2560: go(fixed_row_kernel<ADD, 320, 2>(), 320); return true;
    case 3072: go(fixed_row_kernel<ADD, 256, 3>(), 256); return true;
    case 3584: go(fixed_row_kernel<ADD, 448, 2>(), 448); return true;
    case 3840: go(fixed_row_kernel<ADD, 960, 1>(), 960); return true;
    case 5120: go(fixed_row_kernel<ADD, 640, 2>(), 640); return true;
    case 8192: go(fixed_row_kernel<ADD, 512, 4>(), 512); return true;
  }
  const int chunks = L.dim / 4;  // a multiple of 64: whole waves
  if (chunks % 128 == 0 && chunks / 2 <= 1024)
    go(fixed_row_kernel<ADD, 0, 2>(), chunks / 2);
  else if (chunks <= 1024)
    go(fixed_row_kernel<ADD, 0, 1>(), chunks);
  else
    return false;
  return true;
}

void launch_fused_add_rmsnorm(float *o, float *residual, const float *add, const float *weight, int rows, int dim,
                              float eps, hipStream_t stream) {
  const RowLaunch L{rows, dim, stream};
  if (!launch_fixed_row<true>(L, o, residual, add, weight, eps))
    dispatch_rows<AddNormOp>(L, o, residual, add, weight, eps);
}

void launch_rmsnorm(float *o, const float *x, const float *weight, int rows, int dim, float eps, hipStream_t stream) {
  const RowLaunch L{rows, dim, stream};
  if (!launch_fixed_row<false>(L, o, const_cast<float *>(x), nullptr, weight, eps))
    dispatch_rows<NormOp>(L, o, const_cast<float *>(x), weight, eps);
}

void launch_rmsnorm_quantize(int8_t *q, float *q_s, float *x, const float *add, const float *weight, int rows,
                             int dim, int gs, float eps, hipStream_t stream) {
  // The 16-elements-per-thread kernel needs the 32 chain lanes (dim >= 512), whole
  // 32-element blocks, 16-byte aligned codes and at most 64 KiB of LDS (5 bytes per element).
  if (dim % 32 == 0 && dim >= 512 && dim <= 12288 && ((uintptr_t)q & 15u) == 0) {
    const dim3 grid(rows), block(dim / 16);
    const unsigned lds = (unsigned)(dim + dim / 4) * sizeof(float);
    auto go = [&](auto kernel) { enqueue(kernel, grid, block, lds, stream, q, q_s, x, add, weight, dim, eps); };
    const bool g32 = gs == 32;
    auto go_tpb = [&](auto tpb) {
      constexpr int TPB = decltype(tpb)::value;
      if (add)
        go(g32 ? norm_q8_row16_kernel<TPB, 32, true> : norm_q8_row16_kernel<TPB, 64, true>);
      else
        go(g32 ? norm_q8_row16_kernel<TPB, 32, false> : norm_q8_row16_kernel<TPB, 64, false>);
    };
    // The block size compiled in for the common model widths: 0.2 to 2.7 points
    // of the HBM peak above the run-time block size at [8192, dim].
    switch (dim) {
      case 2048: go_tpb(std::integral_constant<int, 128>{}); break;
      case 2560: go_tpb(std::integral_constant<int, 160>{}); break;
      case 3072: go_tpb(std::integral_constant<int, 192>{}); break;
      case 3584: go_tpb(std::integral_constant<int, 224>{}); break;
      case 3840: go_tpb(std::integral_constant<int, 240>{}); break;
      case 4096: go_tpb(std::integral_constant<int, 256>{}); break;
      case 5120: go_tpb(std::integral_constant<int, 320>{}); break;
      case 6144: go_tpb(std::integral_constant<int, 384>{}); break;
      case 8192: go_tpb(std::integral_constant<int, 512>{}); break;
      default: go_tpb(std::integral_constant<int, 0>{}); break;
    }
    return;
  }
  dispatch_rows<NormQ8Op>(RowLaunch{rows, dim, stream}, q, q_s, x, add, weight, eps, gs);
}

}  // namespace v7g
