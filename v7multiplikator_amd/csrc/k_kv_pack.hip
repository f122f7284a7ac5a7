// k_kv_pack.hip -- K/V rows binary32 -> binary16 for the KV cache, gfx950.
//
// Reference: v7s_kv_pack_f16(dest, src, count), src/asm/kv_f16c.inc:12-52
// (internal in v7): dest[i] = vcvtps2ph(src[i], nearest-even) for one row of
// count floats, called once per token for the K row and the V row after RoPE
// (src/asm/forward_q8.inc:345-358, prefill_q8.inc:157-171, with the cache
// row at cache + loff + pos*kv_dim).  Here one launch packs `rows` rows with
// independent strides: blockIdx.y walks the rows (no per-thread division), and
// each thread converts one float4 (a streaming 16-byte load) into four
// binary16 values (one streaming 8-byte store).
#include "v7g_device.h"
#include "v7g_internal.h"

namespace v7g {

__global__ __launch_bounds__(256) void kv_pack_f16_kernel(uint16_t *dst, long long dst_stride, const float *src,
                                                          long long src_stride, unsigned chunks_per_row,
                                                          unsigned rows) {
  const unsigned j = blockIdx.x * 256u + threadIdx.x;
  if (j >= chunks_per_row) return;
  for (unsigned r = blockIdx.y; r < rows; r += gridDim.y) {
    const float4 v = ld_stream4(src + (long long)r * src_stride + 4 * j);
    st_stream_u2(reinterpret_cast<uint32_t *>(dst + (long long)r * dst_stride + 4 * j), pack4_f16(v));
  }
}

void launch_kv_pack_f16(uint16_t *dst, long long dst_stride, const float *src, long long src_stride, int rows,
                        int row_len, hipStream_t stream) {
  const unsigned cpr = (unsigned)row_len / 4u;
  const dim3 grid((cpr + 255u) / 256u, (unsigned)(rows < 65535 ? rows : 65535));
  enqueue(kv_pack_f16_kernel, grid, dim3(256), 0, stream, dst, dst_stride, src, src_stride, cpr, (unsigned)rows);
}

}  // namespace v7g
