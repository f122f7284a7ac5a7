// k_embedding.hip -- Q8 embedding-row gather + dequant for gfx950.
//
// Reference: v7s_embedding_row (src/asm/forward.inc:13-42), one token row per
// call: out[i] = (float)q[token*dim + i] * s[(token*dim >> 6) + i/64], an exact
// int8 -> f32 conversion followed by one multiply.  Here one launch gathers all
// tokens of a batch; the result is bit-identical by construction.
//
// Layout: a 256-thread block covers 4096 codes (1024 dwords) of one row; lane
// l loads dwords l, l+256, l+512, l+768 of that stretch (four codes each, each
// load one coalesced 1 KiB access per wave, all four issued before any
// convert) with the 64-code group's scale, and stores four floats per dword
// (coalesced 4 KiB dwordx4 stores per wave).  The codes stream past the
// caches (nontemporal loads: each table row is read once); the scales and the
// output use ordinary accesses.  Ordinary stores leave the output rows in the
// caches for the layer that reads them next; inside the per-layer chain at
// T = 8192 they took the gather from 31.0 to 27.7 us with the same chain total
// as streaming stores (the lines drain while the next kernels run).  Rows of
// dim % 4096 == 0 take dim/4096 such blocks.  Any other row up to 8192 codes is
// one block of ceil(dim/16) threads rounded up to whole waves, so that no
// wave of the launch is left without codes (with 256-thread blocks a row of
// 5120 codes took a second block of which three waves had nothing to do:
// 51.7% of the HBM peak against 63.2% at [8192 ids, 5120]; 56.2% against 60.6%
// at 2048).  Wider rows take ceil(dim/4096) blocks of 256 threads.  A thread
// whose dwords run past the row clamps its loads and predicates its stores.
#include "v7g_device.h"
#include "v7g_internal.h"

namespace v7g {

constexpr unsigned kEmbDwords = 4;  // dwords (4 codes each) per thread

__global__ __launch_bounds__(512) void embedding_gather_q8_kernel(float *__restrict__ out,
                                                                  const int32_t *__restrict__ ids,
                                                                  unsigned blocks_per_row,
                                                                  const int8_t *__restrict__ table_q,
                                                                  const float *__restrict__ table_s, int dim,
                                                                  int vocab) {
  const unsigned tb = blockDim.x;
  const unsigned t = blockIdx.x / blocks_per_row;
  const unsigned w0 = (blockIdx.x - t * blocks_per_row) * (tb * kEmbDwords) + threadIdx.x;
  const unsigned dw = (unsigned)dim >> 2;  // dwords per row
  const int id = ids ? ids[t] : (int)t;    // no id array: row t of the table
  float *dst = out + (size_t)t * dim;
  if ((unsigned)id >= (unsigned)vocab) {
    // An id outside the table cannot be read; its row is written as zeros.
#pragma unroll
    for (unsigned j = 0; j < kEmbDwords; ++j) {
      const unsigned w = w0 + tb * j;
      if (w < dw) *reinterpret_cast<float4 *>(dst + 4 * w) = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    return;
  }
  const size_t base = (size_t)id * (size_t)dim;
  const uint32_t *src = reinterpret_cast<const uint32_t *>(table_q + base);
  const float *sc = table_s + (base >> 6);
  uint32_t q[kEmbDwords];
  float s[kEmbDwords];
#pragma unroll
  for (unsigned j = 0; j < kEmbDwords; ++j) {
    const unsigned w = w0 + tb * j;
    const unsigned wc = w < dw ? w : dw - 1;
    q[j] = ld_stream_u32(src + wc);
    s[j] = sc[wc >> 4];
  }
#pragma unroll
  for (unsigned j = 0; j < kEmbDwords; ++j) {
    const unsigned w = w0 + tb * j;
    const uint32_t u = q[j];
    const float4 v = make_float4((float)((int32_t)(u << 24) >> 24) * s[j], (float)((int32_t)(u << 16) >> 24) * s[j],
                                 (float)((int32_t)(u << 8) >> 24) * s[j], (float)((int32_t)u >> 24) * s[j]);
    if (w < dw) *reinterpret_cast<float4 *>(dst + 4 * w) = v;
  }
}

void launch_embedding_gather(float *out, const int32_t *ids, int n_tokens, const int8_t *table_q,
                             const float *table_s, int dim, int vocab, hipStream_t stream) {
  const unsigned dw = (unsigned)dim / 4u;
  unsigned tb = 256u, bpr = (dw + 256u * kEmbDwords - 1u) / (256u * kEmbDwords);
  if (dim % 4096 != 0 && dim <= 8192) {
    tb = (dw + kEmbDwords - 1u) / kEmbDwords;
    tb = (tb + 63u) / 64u * 64u;  // whole waves, at most 512 threads
    bpr = 1u;
  }
  enqueue(embedding_gather_q8_kernel, dim3((unsigned)n_tokens * bpr), dim3(tb), 0, stream, out, ids, bpr, table_q,
          table_s, dim, vocab);
}

}  // namespace v7g
