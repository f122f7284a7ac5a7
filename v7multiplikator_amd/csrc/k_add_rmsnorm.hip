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
#include "v7g_device.h"
#include "v7g_internal.h"

namespace v7g {

// One row.  ADD: the input is residual + add (residual updated in place),
// else x.  QGS == 0: o = (s*x)*w; QGS = 32 or 64: the normalised row is
// quantized in groups of QGS (codes q, scales q_s) and o is not written.
// o may alias residual (the row then ends as o, as in the reference).
template <int TPR, int KMAX, bool ADD, int QGS>
__device__ __forceinline__ void rms_row(float *o, int8_t *q, float *q_s, float *xin, const float *add,
                                        const float *weight, int dim, float eps) {
  extern __shared__ float row[];
  const int tid = threadIdx.x;
  const size_t r = blockIdx.x;
  float *xr = xin + r * (size_t)dim;

  // Pass 1: load the row (and add), stage it in LDS.
  float4 x[KMAX], b[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int i = 4 * (tid + k * TPR);
    if (i < dim) {
      x[k] = ld_stream4(xr + i);
      if constexpr (ADD) b[k] = ld_stream4(add + r * (size_t)dim + i);
    }
  }
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int i = 4 * (tid + k * TPR);
    if (i < dim) {
      if constexpr (ADD) {
        x[k] = make_float4(x[k].x + b[k].x, x[k].y + b[k].y, x[k].z + b[k].z, x[k].w + b[k].w);
        st_stream4(xr + i, x[k]);
      }
      *reinterpret_cast<float4 *>(row + i) = x[k];
    }
  }
  __syncthreads();

  if (tid < 64) {
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
  const float s = row[0];

  // Pass 2: n = (s * x) * w, then either stored or quantized.
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int i = 4 * (tid + k * TPR);
    const bool live = i < dim;
    float4 n = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) {
      const float4 w = *reinterpret_cast<const float4 *>(weight + i);
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

template <int TPR, int KMAX>
__global__ __launch_bounds__(TPR) void fused_add_rmsnorm_kernel(float *o, float *residual, const float *add,
                                                                const float *weight, int dim, float eps) {
  rms_row<TPR, KMAX, true, 0>(o, nullptr, nullptr, residual, add, weight, dim, eps);
}

template <int TPR, int KMAX>
__global__ __launch_bounds__(TPR) void rmsnorm_kernel(float *o, float *x, const float *weight, int dim, float eps) {
  rms_row<TPR, KMAX, false, 0>(o, nullptr, nullptr, x, nullptr, weight, dim, eps);
}

template <int TPR, int KMAX, int QGS>
__global__ __launch_bounds__(TPR) void rmsnorm_quantize_kernel(int8_t *q, float *q_s, float *x, const float *weight,
                                                               int dim, float eps) {
  rms_row<TPR, KMAX, false, QGS>(nullptr, q, q_s, x, nullptr, weight, dim, eps);
}

template <int TPR, int KMAX, int QGS>
__global__ __launch_bounds__(TPR) void add_rmsnorm_quantize_kernel(int8_t *q, float *q_s, float *residual,
                                                                   const float *add, const float *weight, int dim,
                                                                   float eps) {
  rms_row<TPR, KMAX, true, QGS>(nullptr, q, q_s, residual, add, weight, dim, eps);
}

// Chooses threads per row and float4 chunks per thread for dim <= 16384
// (validated by the caller) and launches one workgroup per row.
struct RowLaunch {
  int rows, dim;
  hipStream_t stream;
  size_t lds() const { return (size_t)dim * sizeof(float); }
};

template <template <int, int> class Op, typename... A>
static void dispatch_rows(const RowLaunch &L, A... args) {
  if (L.dim <= 256)
    Op<64, 1>::launch(L, args...);
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
    enqueue((fused_add_rmsnorm_kernel<TPR, KMAX>), dim3(L.rows), dim3(TPR), L.lds(), L.stream, o,
                       residual, add, weight, L.dim, eps);
  }
};

template <int TPR, int KMAX>
struct NormOp {
  static void launch(const RowLaunch &L, float *o, float *x, const float *weight, float eps) {
    enqueue((rmsnorm_kernel<TPR, KMAX>), dim3(L.rows), dim3(TPR), L.lds(), L.stream, o, x, weight, L.dim,
                       eps);
  }
};

template <int TPR, int KMAX>
struct NormQ8Op {
  static void launch(const RowLaunch &L, int8_t *q, float *q_s, float *x, const float *add, const float *weight,
                     float eps, int gs) {
    if (add) {
      if (gs == 32)
        enqueue((add_rmsnorm_quantize_kernel<TPR, KMAX, 32>), dim3(L.rows), dim3(TPR), L.lds(), L.stream,
                           q, q_s, x, add, weight, L.dim, eps);
      else
        enqueue((add_rmsnorm_quantize_kernel<TPR, KMAX, 64>), dim3(L.rows), dim3(TPR), L.lds(), L.stream,
                           q, q_s, x, add, weight, L.dim, eps);
    } else {
      if (gs == 32)
        enqueue((rmsnorm_quantize_kernel<TPR, KMAX, 32>), dim3(L.rows), dim3(TPR), L.lds(), L.stream, q,
                           q_s, x, weight, L.dim, eps);
      else
        enqueue((rmsnorm_quantize_kernel<TPR, KMAX, 64>), dim3(L.rows), dim3(TPR), L.lds(), L.stream, q,
                           q_s, x, weight, L.dim, eps);
    }
  }
};

void launch_fused_add_rmsnorm(float *o, float *residual, const float *add, const float *weight, int rows, int dim,
                              float eps, hipStream_t stream) {
  dispatch_rows<AddNormOp>(RowLaunch{rows, dim, stream}, o, residual, add, weight, eps);
}

void launch_rmsnorm(float *o, const float *x, const float *weight, int rows, int dim, float eps, hipStream_t stream) {
  dispatch_rows<NormOp>(RowLaunch{rows, dim, stream}, o, const_cast<float *>(x), weight, eps);
}

void launch_rmsnorm_quantize(int8_t *q, float *q_s, float *x, const float *add, const float *weight, int rows,
                             int dim, int gs, float eps, hipStream_t stream) {
  dispatch_rows<NormQ8Op>(RowLaunch{rows, dim, stream}, q, q_s, x, add, weight, eps, gs);
}

}  // namespace v7g
