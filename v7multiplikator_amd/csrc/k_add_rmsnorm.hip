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
// This kernel reproduces that order exactly, so its output is bit-identical:
// one wave per row; pass 1 streams the row with dwordx4 loads and stages the
// updated residual in LDS; 32 lanes then replay the 32 FMA chains (lane
// 8q + j is accumulator q, YMM lane j) from LDS, conflict-free; the five-step
// xor exchange below is exactly the (A+B)+(C+D) + HADD_YMM pairing; pass 2
// reads the row back from LDS.
#include "v7g_device.h"
#include "v7g_internal.h"

namespace v7g {

// o may alias residual (the row then ends as o, as in the reference); no
// pointer is declared __restrict__.
__global__ __launch_bounds__(64) void fused_add_rmsnorm_kernel(float *o, float *residual, const float *add,
                                                               const float *weight, int dim, float eps) {
  extern __shared__ float row[];
  const int lane = threadIdx.x;
  const size_t r = blockIdx.x;
  float *res = residual + r * (size_t)dim;
  const float *ad = add + r * (size_t)dim;
  float *out = o + r * (size_t)dim;

  // Pass 1: r = residual + add, written back and staged in LDS.
  int i = lane * 4;
  for (; i + 3 * 256 < dim; i += 4 * 256) {
    float4 a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) a[u] = *reinterpret_cast<const float4 *>(res + i + u * 256);
#pragma unroll
    for (int u = 0; u < 4; ++u) b[u] = *reinterpret_cast<const float4 *>(ad + i + u * 256);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float4 x = make_float4(a[u].x + b[u].x, a[u].y + b[u].y, a[u].z + b[u].z, a[u].w + b[u].w);
      *reinterpret_cast<float4 *>(res + i + u * 256) = x;
      *reinterpret_cast<float4 *>(row + i + u * 256) = x;
    }
  }
  for (; i < dim; i += 256) {
    float4 a = *reinterpret_cast<const float4 *>(res + i);
    float4 b = *reinterpret_cast<const float4 *>(ad + i);
    float4 x = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
    *reinterpret_cast<float4 *>(res + i) = x;
    *reinterpret_cast<float4 *>(row + i) = x;
  }
  __syncthreads();

  // The 32 FMA chains: lane v = 8q + j is YMM accumulator q (A..D), lane j.
  float acc = 0.0f;
  if (lane < 32) {
    const int q = lane >> 3, j = lane & 7;
    const int blocks = dim >> 3, left = blocks & 3, groups = blocks >> 2;
    if (q == 0)
      for (int b = 0; b < left; ++b) {
        float x = row[8 * b + j];
        acc = __builtin_fmaf(x, x, acc);
      }
    const float *p = row + 8 * (left + q) + j;
#pragma unroll 8
    for (int g = 0; g < groups; ++g) {
      float x = p[32 * g];
      acc = __builtin_fmaf(x, x, acc);
    }
  }
  // (A+B), (C+D): xor 8; then their sum: xor 16; HADD_YMM: xor 4, xor 1, xor 2.
  acc = acc + xor_f(acc, 8);
  acc = acc + xor_f(acc, 16);
  acc = acc + xor_f(acc, 4);
  acc = acc + xor_f(acc, 1);
  acc = acc + xor_f(acc, 2);
  const float ss = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, acc)));
  const float s = rms_scale(ss, (float)dim, eps);

  // Pass 2: o = (s * r) * w.
  for (i = lane * 4; i < dim; i += 256) {
    float4 x = *reinterpret_cast<const float4 *>(row + i);
    float4 w = *reinterpret_cast<const float4 *>(weight + i);
    float4 y = make_float4((s * x.x) * w.x, (s * x.y) * w.y, (s * x.z) * w.z, (s * x.w) * w.w);
    *reinterpret_cast<float4 *>(out + i) = y;
  }
}

void launch_fused_add_rmsnorm(float *o, float *residual, const float *add, const float *weight, int rows, int dim,
                              float eps, hipStream_t stream) {
  size_t lds = (size_t)dim * sizeof(float);
  hipLaunchKernelGGL(fused_add_rmsnorm_kernel, dim3(rows), dim3(64), lds, stream, o, residual, add, weight, dim, eps);
}

}  // namespace v7g
