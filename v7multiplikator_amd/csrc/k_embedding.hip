// k_embedding.hip -- Q8 embedding-row gather + dequant for gfx950.
//
// Reference: v7s_embedding_row (src/asm/forward.inc:13-42), one token row per
// call: out[i] = (float)q[token*dim + i] * s[(token*dim >> 6) + i/64], an exact
// int8 -> f32 conversion followed by one multiply.  Here one launch gathers all
// tokens of a batch; the result is bit-identical by construction.
//
// Layout: each thread owns 16 consecutive codes of one row (one dwordx4 load,
// always inside one 64-code scale group) and writes 16 floats.  A 256-thread
// block covers 4096 codes, i.e. exactly one row at dim 4096.
#include "v7g_device.h"
#include "v7g_internal.h"

namespace v7g {

__global__ __launch_bounds__(256) void embedding_gather_q8_kernel(float *__restrict__ out,
                                                                  const int32_t *__restrict__ ids, uint32_t n_chunks,
                                                                  uint32_t chunks_per_row,
                                                                  const int8_t *__restrict__ table_q,
                                                                  const float *__restrict__ table_s, int dim,
                                                                  int vocab) {
  uint32_t c = blockIdx.x * 256u + threadIdx.x;
  if (c >= n_chunks) return;
  uint32_t t = c / chunks_per_row;
  uint32_t j = c - t * chunks_per_row;
  int id = ids ? ids[t] : (int)t;  // no id array: row t of the table
  float4 *dst = reinterpret_cast<float4 *>(out + (size_t)t * dim + 16u * j);
  if ((unsigned)id >= (unsigned)vocab) {
    // An id outside the table cannot be read; its row is written as zeros.
    float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    dst[0] = z; dst[1] = z; dst[2] = z; dst[3] = z;
    return;
  }
  size_t base = (size_t)id * (size_t)dim;
  uint4 w = *reinterpret_cast<const uint4 *>(table_q + base + 16u * j);
  float s = table_s[(base >> 6) + ((16u * j) >> 6)];
  uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t u = words[k];
    float4 v;
    v.x = (float)((int32_t)(u << 24) >> 24) * s;
    v.y = (float)((int32_t)(u << 16) >> 24) * s;
    v.z = (float)((int32_t)(u << 8) >> 24) * s;
    v.w = (float)((int32_t)u >> 24) * s;
    dst[k] = v;
  }
}

void launch_embedding_gather(float *out, const int32_t *ids, int n_tokens, const int8_t *table_q,
                             const float *table_s, int dim, int vocab, hipStream_t stream) {
  uint32_t cpr = (uint32_t)dim / 16u;
  uint32_t n_chunks = (uint32_t)n_tokens * cpr;
  uint32_t blocks = (n_chunks + 255u) / 256u;
  hipLaunchKernelGGL(embedding_gather_q8_kernel, dim3(blocks), dim3(256), 0, stream, out, ids, n_chunks, cpr, table_q,
                     table_s, dim, vocab);
}

}  // namespace v7g
