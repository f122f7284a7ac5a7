// k_embedding.hip -- Q8 embedding-row gather + dequant for gfx950.
//
// Reference: v7s_embedding_row (src/asm/forward.inc:13-42), one token row per
// call: out[i] = (float)q[token*dim + i] * s[(token*dim >> 6) + i/64], an exact
// int8 -> f32 conversion followed by one multiply.  Here one launch gathers all
// tokens of a batch; the result is bit-identical by construction.
//
// Flat pieces (rows of dim >= 256 codes).  The output of a launch, n_tokens
// rows of dim floats, is taken as one array of n_tokens*dim/4 "dwords" (four
// codes in, one float4 out).  Piece p is the 512 dwords [512p, 512p + 512).
// Workgroup b = 8g + x (512 threads) handles pieces 8*(2g) + x and
// 8*(2g+1) + x, one dword per lane in each: every id load first (scalar
// loads), then the four code and scale loads of the lane, then two float4
// streaming stores, each a coalesced 1 KiB per wave.  A wave's 64 dwords lie
// in at most two rows (dim/4 >= 64): the wave reads both ids and each lane
// takes its own; the row index is the dword index times a 64-bit reciprocal
// of dim/4 (exact for every 32-bit dividend).  The codes stream past the
// caches (nontemporal loads, each table row is read once) and so does the
// output (nontemporal stores reach HBM within the kernel instead of leaving
// dirty lines for the next kernel to write back).
//
// Measured at [8192 ids, 151936 x 4096], launches back to back with buffers
// rotating past the 256 MiB Infinity Cache, one MI355X: 29.9 us (71.0% of the
// HBM peak) against 32.8 us for the earlier form (one 256-thread workgroup per
// 4096 codes of a row, four dwords per lane, ordinary stores).  What moved it:
// two pieces per workgroup (one: 34.3 us; three: 32.1), 512 threads (256:
// 30.1 us; 1024: 30.2), scalar id loads (a vector id load ahead of the code
// loads: 38.1 us), streaming stores (ordinary: +2.3 us), all id loads issued
// before the first code load.  The same form at the other model widths:
// 896 codes 9.6 -> 8.8 us, 1536 14.7 -> 13.0, 2560 22.6 -> 19.9, 3584
// 29.7 -> 26.7, 5120 43.5 -> 36.9, 8192 62.8 -> 57.2.
//
// The launch runs the pieces that fill whole groups of 8 workgroups without a
// bounds test; a last group of 8 workgroups covers the rest with one.  Rows
// narrower than 256 codes (and launches of 2^32 dwords or more) take one
// workgroup per row of ceil(dim/16) threads rounded up to whole waves, four
// dwords per thread.
#include "v7g_device.h"
#include "v7g_internal.h"

namespace v7g {

constexpr unsigned kEmbPiece = 512;  // dwords per piece = threads per workgroup
constexpr unsigned kEmbPieces = 2;   // pieces per workgroup
constexpr unsigned kEmbGroup = 8 * kEmbPieces * kEmbPiece;  // dwords covered by 8 consecutive workgroups

__device__ __forceinline__ float4 dequant4(uint32_t u, float s) {
  return make_float4((float)((int32_t)(u << 24) >> 24) * s, (float)((int32_t)(u << 16) >> 24) * s,
                     (float)((int32_t)(u << 8) >> 24) * s, (float)((int32_t)u >> 24) * s);
}

// TAIL: the last group of workgroups, whose dwords may run past the launch's
// rows*dw: their loads are clamped into row 0 and their stores predicated.
template <bool TAIL>
__device__ __forceinline__ void gather_pieces(float *__restrict__ out, const int32_t *__restrict__ ids,
                                              const uint32_t *__restrict__ tq4, const float *__restrict__ ts,
                                              unsigned dw, unsigned long long magic, unsigned rows, int vocab) {
  const unsigned b = blockIdx.x, x = b & 7u, g = b >> 3;
  const unsigned wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const unsigned lane = threadIdx.x & 63u;
  const unsigned total = rows * dw;
  const unsigned sdw = dw >> 4;  // scales per row
  unsigned e0[kEmbPieces], r0[kEmbPieces], b1[kEmbPieces];
  int id0[kEmbPieces], id1[kEmbPieces];
#pragma unroll
  for (unsigned j = 0; j < kEmbPieces; ++j) {
    const unsigned p = 8u * (kEmbPieces * g + j) + x;
    e0[j] = p * kEmbPiece + 64u * wv;  // the wave's first dword
    const unsigned ec = (TAIL && e0[j] >= total) ? total - 1u : e0[j];
    r0[j] = (unsigned)__umul64hi((unsigned long long)ec, magic);  // ec / dw
    b1[j] = (r0[j] + 1u) * dw;                                     // first dword of the next row
    const unsigned r1 = r0[j] + 1u < rows ? r0[j] + 1u : rows - 1u;
    id0[j] = ids ? ids[r0[j]] : (int)r0[j];  // no id array: row r of the table
    id1[j] = ids ? ids[r1] : (int)r1;
  }
  uint32_t q[kEmbPieces];
  float s[kEmbPieces];
  bool ok[kEmbPieces];
#pragma unroll
  for (unsigned j = 0; j < kEmbPieces; ++j) {
    const unsigned e = e0[j] + lane;
    const bool second = e >= b1[j];
    int id = second ? id1[j] : id0[j];
    unsigned d = second ? e - b1[j] : e - r0[j] * dw;  // dword within the row
    if (TAIL && e >= total) id = 0, d = 0;
    // An id outside the table cannot be read; its row is written as zeros.
    ok[j] = (unsigned)id < (unsigned)vocab;
    if (!ok[j]) id = 0;
    q[j] = ld_stream_u32(tq4 + (size_t)(unsigned)id * dw + d);
    s[j] = ts[(size_t)(unsigned)id * sdw + (d >> 4)];
  }
#pragma unroll
  for (unsigned j = 0; j < kEmbPieces; ++j) {
    const unsigned e = e0[j] + lane;
    float4 v = dequant4(q[j], s[j]);
    if (!ok[j]) v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (!TAIL || e < total) st_stream4(out + 4 * (size_t)e, v);
  }
}

__global__ __launch_bounds__(kEmbPiece) void embedding_gather_q8_kernel(float *__restrict__ out,
                                                                        const int32_t *__restrict__ ids,
                                                                        const int8_t *__restrict__ table_q,
                                                                        const float *__restrict__ table_s,
                                                                        unsigned dw, unsigned long long magic,
                                                                        unsigned rows, unsigned full_blocks,
                                                                        int vocab) {
  const uint32_t *tq4 = reinterpret_cast<const uint32_t *>(table_q);
  if (blockIdx.x < full_blocks)
    gather_pieces<false>(out, ids, tq4, table_s, dw, magic, rows, vocab);
  else
    gather_pieces<true>(out, ids, tq4, table_s, dw, magic, rows, vocab);
}

// One workgroup per row: rows narrower than 256 codes, or launches too large
// for 32-bit dword indices.  Four dwords per thread (stride one workgroup);
// rows up to 8192 codes take one workgroup of ceil(dim/16) threads rounded up
// to whole waves, wider rows ceil(dim/4096) workgroups of 256 threads.
constexpr unsigned kRowDwords = 4;

__global__ __launch_bounds__(512) void embedding_gather_rows_kernel(float *__restrict__ out,
                                                                    const int32_t *__restrict__ ids,
                                                                    unsigned blocks_per_row,
                                                                    const int8_t *__restrict__ table_q,
                                                                    const float *__restrict__ table_s, int dim,
                                                                    int vocab) {
  const unsigned tb = blockDim.x;
  const unsigned t = blockIdx.x / blocks_per_row;
  const unsigned w0 = (blockIdx.x - t * blocks_per_row) * (tb * kRowDwords) + threadIdx.x;
  const unsigned dw = (unsigned)dim >> 2;  // dwords per row
  const int id = ids ? ids[t] : (int)t;    // no id array: row t of the table
  float *dst = out + (size_t)t * dim;
  if ((unsigned)id >= (unsigned)vocab) {
#pragma unroll
    for (unsigned j = 0; j < kRowDwords; ++j) {
      const unsigned w = w0 + tb * j;
      if (w < dw) st_stream4(dst + 4 * w, make_float4(0.f, 0.f, 0.f, 0.f));
    }
    return;
  }
  const size_t base = (size_t)id * (size_t)dim;
  const uint32_t *src = reinterpret_cast<const uint32_t *>(table_q + base);
  const float *sc = table_s + (base >> 6);
  uint32_t q[kRowDwords];
  float s[kRowDwords];
#pragma unroll
  for (unsigned j = 0; j < kRowDwords; ++j) {
    const unsigned w = w0 + tb * j;
    const unsigned wc = w < dw ? w : dw - 1;
    q[j] = ld_stream_u32(src + wc);
    s[j] = sc[wc >> 4];
  }
#pragma unroll
  for (unsigned j = 0; j < kRowDwords; ++j) {
    const unsigned w = w0 + tb * j;
    if (w < dw) st_stream4(dst + 4 * w, dequant4(q[j], s[j]));
  }
}

void launch_embedding_gather(float *out, const int32_t *ids, int n_tokens, const int8_t *table_q,
                             const float *table_s, int dim, int vocab, hipStream_t stream) {
  const unsigned dw = (unsigned)dim / 4u;
  const unsigned long long total = (unsigned long long)n_tokens * dw;
  if (dw >= 64u && total + kEmbGroup < (1ull << 32)) {
    const unsigned full_blocks = (unsigned)(total / kEmbGroup) * 8u;
    const unsigned grid = full_blocks + (total % kEmbGroup ? 8u : 0u);
    const unsigned long long magic = ~0ull / dw + 1ull;  // n / dw == umulhi64(n, magic) for every n < 2^32
    enqueue(embedding_gather_q8_kernel, dim3(grid), dim3(kEmbPiece), 0, stream, out, ids, table_q, table_s, dw,
            magic, (unsigned)n_tokens, full_blocks, vocab);
    return;
  }
  unsigned tb = 256u, bpr = (dw + 256u * kRowDwords - 1u) / (256u * kRowDwords);
  if (dim % 4096 != 0 && dim <= 8192) {
    tb = (dw + kRowDwords - 1u) / kRowDwords;
    tb = (tb + 63u) / 64u * 64u;  // whole waves, at most 512 threads
    bpr = 1u;
  }
  enqueue(embedding_gather_rows_kernel, dim3((unsigned)n_tokens * bpr), dim3(tb), 0, stream, out, ids, bpr, table_q,
          table_s, dim, vocab);
}

}  // namespace v7g
