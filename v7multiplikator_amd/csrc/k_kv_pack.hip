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

// The K and V rows of a token batch in one grid (the two v7s_kv_pack_f16
// calls per token of src/asm/forward_q8.inc:345-358): each thread converts
// the same float4 chunk of a token's K row and of its V row (two streaming
// loads issued together, two 8-byte stores), so a workgroup reads the
// token's K and V stretch of the QKV row side by side.  Measured at 8192
// tokens x 1024: 17.7 us against 18.6 us for one thread per chunk of either
// side and 20.6-21.1 us for two launches.  Strides below 2^32 elements go as
// 32-bit arguments (S = unsigned): the arguments then fill 13 dwords, all of
// which the firmware preloads into SGPRs at wave launch, where with 64-bit
// strides the chunk count and the row count come past the 14 preloaded
// dwords and each wave waits for a scalar load of them first.
template <typename S>
__global__ __launch_bounds__(256) void kv_pack2_f16_kernel(uint16_t *k_dst, uint16_t *v_dst, const float *k_src,
                                                           const float *v_src, S k_dst_stride, S v_dst_stride,
                                                           S src_stride, unsigned chunks_per_row, unsigned rows) {
  const unsigned j = blockIdx.x * 256u + threadIdx.x;
  if (j >= chunks_per_row) return;
  for (unsigned r = blockIdx.y; r < rows; r += gridDim.y) {
    const float4 k = ld_stream4(k_src + (long long)r * (long long)src_stride + 4 * j);
    const float4 v = ld_stream4(v_src + (long long)r * (long long)src_stride + 4 * j);
    st_stream_u2(reinterpret_cast<uint32_t *>(k_dst + (long long)r * (long long)k_dst_stride + 4 * j), pack4_f16(k));
    st_stream_u2(reinterpret_cast<uint32_t *>(v_dst + (long long)r * (long long)v_dst_stride + 4 * j), pack4_f16(v));
  }
}

void launch_kv_pack2_f16(uint16_t *k_dst, long long k_dst_stride, uint16_t *v_dst, long long v_dst_stride,
                         const float *k_src, const float *v_src, long long src_stride, int rows, int row_len,
                         hipStream_t stream) {
  const unsigned cpr = (unsigned)row_len / 4u;
  const dim3 grid((cpr + 255u) / 256u, (unsigned)(rows < 65535 ? rows : 65535));
  if (rows <= 1) k_dst_stride = v_dst_stride = src_stride = 0;  // row 0 only: no stride is read
  auto narrow = [](long long v) { return v >= 0 && v <= 0xFFFFFFFFLL; };
  if (narrow(k_dst_stride) && narrow(v_dst_stride) && narrow(src_stride))
    enqueue(kv_pack2_f16_kernel<unsigned>, grid, dim3(256), 0, stream, k_dst, v_dst, k_src, v_src,
            (unsigned)k_dst_stride, (unsigned)v_dst_stride, (unsigned)src_stride, cpr, (unsigned)rows);
  else
    enqueue(kv_pack2_f16_kernel<long long>, grid, dim3(256), 0, stream, k_dst, v_dst, k_src, v_src, k_dst_stride,
            v_dst_stride, src_stride, cpr, (unsigned)rows);
}

void launch_kv_pack_f16(uint16_t *dst, long long dst_stride, const float *src, long long src_stride, int rows,
                        int row_len, hipStream_t stream) {
  const unsigned cpr = (unsigned)row_len / 4u;
  const dim3 grid((cpr + 255u) / 256u, (unsigned)(rows < 65535 ? rows : 65535));
  enqueue(kv_pack_f16_kernel, grid, dim3(256), 0, stream, dst, dst_stride, src, src_stride, cpr, (unsigned)rows);
}

}  // namespace v7g
