// k_kv_pack.hip -- K/V rows binary32 -> binary16 for the KV cache, gfx950.
//
// Reference: v7s_kv_pack_f16(dest, src, count), src/asm/kv_f16c.inc:12-52
// (internal in v7): dest[i] = vcvtps2ph(src[i], nearest-even) for one row of
// count floats, called once per token for the K row and the V row after RoPE
// (src/asm/forward_q8.inc:345-358, prefill_q8.inc:157-171, with the cache
// row at cache + loff + pos*kv_dim).  Here one launch packs `rows` rows with
// independent strides: each thread converts one float4 (a streaming 16-byte
// load) into four binary16 values (one streaming 8-byte store).
#include "v7g_device.h"
#include "v7g_internal.h"

namespace v7g {

__global__ __launch_bounds__(256) void kv_pack_f16_kernel(uint16_t *dst, long long dst_stride, const float *src,
                                                          long long src_stride, unsigned chunks_per_row,
                                                          unsigned long long n_chunks) {
  const unsigned long long c = (unsigned long long)blockIdx.x * 256u + threadIdx.x;
  if (c >= n_chunks) return;
  const unsigned long long r = c / chunks_per_row;
  const unsigned j = (unsigned)(c - r * chunks_per_row);
  const float4 v = ld_stream4(src + r * src_stride + 4 * j);
  st_stream_u2(reinterpret_cast<uint32_t *>(dst + r * dst_stride + 4 * j), pack4_f16(v));
}

void launch_kv_pack_f16(uint16_t *dst, long long dst_stride, const float *src, long long src_stride, int rows,
                        int row_len, hipStream_t stream) {
  const unsigned cpr = (unsigned)row_len / 4u;
  const unsigned long long n = (unsigned long long)rows * cpr;
  const unsigned blocks = (unsigned)((n + 255) / 256);
  enqueue(kv_pack_f16_kernel, dim3(blocks), dim3(256), 0, stream, dst, dst_stride, src, src_stride, cpr,
                     n);
}

}  // namespace v7g
