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
// and o move as streaming loads and stores, the weight row stays cached.  The updated
// residual also goes to LDS, where 32 lanes of wave 0 replay the 32 FMA
// chains (lane 8q + j is accumulator q, YMM lane j), conflict-free; the
// five-step xor exchange below is exactly the (A+B)+(C+D) + HADD_YMM pairing.
#include "v7g_device.h"
#include "v7g_internal.h"

namespace v7g {

// o may alias residual (the row then ends as o, as in the reference); no
// pointer is declared __restrict__.
template <int TPR, int KMAX>
__global__ __launch_bounds__(TPR) void fused_add_rmsnorm_kernel(float *o, float *residual, const float *add,
                                                                const float *weight, int dim, float eps) {
  extern __shared__ float row[];
  const int tid = threadIdx.x;
  const size_t r = blockIdx.x;
  float *res = residual + r * (size_t)dim;
  const float *ad = add + r * (size_t)dim;
  float *out = o + r * (size_t)dim;

  // Pass 1: r = residual + add, written back and staged in LDS.
  float4 x[KMAX], b[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int i = 4 * (tid + k * TPR);
    if (i < dim) {
      x[k] = ld_stream4(res + i);
      b[k] = ld_stream4(ad + i);
    }
  }
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int i = 4 * (tid + k * TPR);
    if (i < dim) {
      x[k] = make_float4(x[k].x + b[k].x, x[k].y + b[k].y, x[k].z + b[k].z, x[k].w + b[k].w);
      st_stream4(res + i, x[k]);
      *reinterpret_cast<float4 *>(row + i) = x[k];
    }
  }
  __syncthreads();

  if (tid < 64) {
    // The 32 FMA chains: lane v = 8q + j is YMM accumulator q (A..D), lane j.
    float acc = 0.0f;
    if (tid < 32) {
      const int q = tid >> 3, j = tid & 7;
      const int blocks = dim >> 3, left = blocks & 3, groups = blocks >> 2;
      if (q == 0)
        for (int bb = 0; bb < left; ++bb) {
          const float v = row[8 * bb + j];
          acc = __builtin_fmaf(v, v, acc);
        }
      const float *p = row + 8 * (left + q) + j;
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

  // Pass 2: o = (s * r) * w.
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int i = 4 * (tid + k * TPR);
    if (i < dim) {
      const float4 w = *reinterpret_cast<const float4 *>(weight + i);
      st_stream4(out + i, make_float4((s * x[k].x) * w.x, (s * x[k].y) * w.y, (s * x[k].z) * w.z, (s * x[k].w) * w.w));
    }
  }
}

template <int TPR, int KMAX>
static void launch_rows(float *o, float *residual, const float *add, const float *weight, int rows, int dim, float eps,
                        hipStream_t stream) {
  const size_t lds = (size_t)dim * sizeof(float);
  hipLaunchKernelGGL((fused_add_rmsnorm_kernel<TPR, KMAX>), dim3(rows), dim3(TPR), lds, stream, o, residual, add,
                     weight, dim, eps);
}

void launch_fused_add_rmsnorm(float *o, float *residual, const float *add, const float *weight, int rows, int dim,
                              float eps, hipStream_t stream) {
  // dim <= 16384 (validated by the caller): at most 16 float4 per thread.
  if (dim <= 256)
    launch_rows<64, 1>(o, residual, add, weight, rows, dim, eps, stream);
  else if (dim <= 1024)
    launch_rows<256, 1>(o, residual, add, weight, rows, dim, eps, stream);
  else if (dim <= 2048)
    launch_rows<256, 2>(o, residual, add, weight, rows, dim, eps, stream);
  else if (dim <= 4096)
    launch_rows<256, 4>(o, residual, add, weight, rows, dim, eps, stream);
  else if (dim <= 8192)
    launch_rows<256, 8>(o, residual, add, weight, rows, dim, eps, stream);
  else
    launch_rows<256, 16>(o, residual, add, weight, rows, dim, eps, stream);
}

}  // namespace v7g
