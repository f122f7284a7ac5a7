// k_selfcheck.hip -- exhaustive check, on the running device, of the three
// arithmetic identities the hot kernels rely on (v7g_device.h):
//   0. rcp_rn(d) == 1.0f / d          for every d in [2^-126, 2^123)
//   1. div127_rn(x) == x / 127.0f     for every finite x >= 127 * 2^-126
//   2. sigmoid_v7(g) == the same sequence with max/min clamp and IEEE
//      division (EVAL_SIGMOID as written, src/asm/v7_macros.inc:98-160) for
//      every non-NaN binary32 g;
//   3. f16_bits(f) == a software binary32 -> binary16 round-to-nearest-even
//      (the rounding of vcvtps2ph imm 0, src/asm/kv_f16c.inc) for every
//      non-NaN binary32 f; a NaN must give a binary16 NaN.
// Each case walks its whole range of bit patterns (about 2^31, 2^31, 2^32 and
// 2^32 values), a few milliseconds of GPU time.  Results are per-block counts in
// caller-visible device memory, summed on the host.
#include <mutex>
#include <vector>

#include "v7g_device.h"
#include "v7g_internal.h"

namespace v7g {

// EVAL_SIGMOID with the reference's operations one for one: vmaxps/vminps
// clamp and vdivps.
__device__ __forceinline__ float sigmoid_ieee(float g) {
  const float log2e = 1.4426950408889634f;
  float x = -g;
  x = __builtin_fmaxf(x, -80.0f);
  x = __builtin_fminf(x, 80.0f);
  float fx = x * log2e;
  float ip = __builtin_rintf(fx);
  float fp = fx - ip;
  float p = bits_f(0x3AADD303u);
  p = __builtin_fmaf(fp, p, bits_f(0x3C1E7411u));
  p = __builtin_fmaf(fp, p, bits_f(0x3D635B9Bu));
  p = __builtin_fmaf(fp, p, bits_f(0x3E75FCE0u));
  p = __builtin_fmaf(fp, p, bits_f(0x3F317215u));
  p = __builtin_fmaf(fp, p, 1.0f);
  float e = __builtin_ldexpf(p, (int)ip);
  return 1.0f / (e + 1.0f);
}

// binary32 -> binary16, round to nearest even, in integer arithmetic.
__device__ __forceinline__ uint32_t f16_bits_sw(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t exp = (u >> 23) & 0xFFu;
  const uint32_t man = u & 0x7FFFFFu;
  if (exp == 0xFFu) return sign | 0x7C00u | (man ? 0x0200u : 0u);
  const int e = (int)exp - 112;  // binary16 biased exponent: exp - 127 + 15
  if (e >= 31) return sign | 0x7C00u;
  if (e <= 0) {
    if (e < -10) return sign;
    const uint32_t m = man | 0x800000u;
    const int shift = 14 - e;
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    return sign | q;
  }
  uint32_t q = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u;
  return sign | q;
}

constexpr int kCheckBlocks = 4096;
constexpr int kChecks = 4;

// Mismatches of identity `which` among this thread's share of patterns lo .. lo+count-1.
__device__ __forceinline__ unsigned long long count_mismatches(int which, uint64_t lo, uint64_t count) {
  unsigned long long bad = 0;
  const uint64_t stride = (uint64_t)gridDim.x * 256u;
  for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < count; i += stride) {
    const float v = bits_f((uint32_t)(lo + i));
    float fast, exact;
    if (which == 0) {
      fast = rcp_rn(v);
      exact = 1.0f / v;
    } else if (which == 1) {
      fast = div127_rn(v);
      exact = v / 127.0f;
    } else if (which == 2) {
      if (v != v) continue;
      fast = sigmoid_v7(v);
      exact = sigmoid_ieee(v);
    } else {
      const uint32_t hw = f16_bits(v);
      if (v != v) {
        bad += (hw & 0x7C00u) != 0x7C00u || (hw & 0x03FFu) == 0u;  // must be a binary16 NaN
        continue;
      }
      bad += hw != f16_bits_sw(v);
      continue;
    }
    bad += __builtin_bit_cast(uint32_t, fast) != __builtin_bit_cast(uint32_t, exact);
  }
  return bad;
}

// The workgroup's total (every thread must call it).
__device__ __forceinline__ unsigned long long block_total(unsigned long long bad) {
  __shared__ unsigned long long part[256];
  part[threadIdx.x] = bad;
  __syncthreads();
  for (int h = 128; h > 0; h >>= 1) {
    if (threadIdx.x < h) part[threadIdx.x] += part[threadIdx.x + h];
    __syncthreads();
  }
  return part[0];
}

// One count per workgroup in block_counts[blockIdx.x].
__global__ __launch_bounds__(256) void arith_check_kernel(int which, uint64_t lo, uint64_t count,
                                                          unsigned long long *block_counts) {
  const unsigned long long total = block_total(count_mismatches(which, lo, count));
  if (threadIdx.x == 0) block_counts[blockIdx.x] = total;
}

// Every workgroup adds its count to *counter (cleared by the caller first).
__global__ __launch_bounds__(256) void arith_count_kernel(int which, uint64_t lo, uint64_t count,
                                                          unsigned long long *counter) {
  const unsigned long long total = block_total(count_mismatches(which, lo, count));
  if (threadIdx.x == 0 && total) atomicAdd(counter, total);
}

__global__ void clear_counters_kernel(unsigned long long *c, int n) {
  if ((int)threadIdx.x < n) c[threadIdx.x] = 0;
}

struct CheckRange {
  uint64_t lo, hi;
};
// The patterns of each identity.
constexpr CheckRange kRanges[kChecks] = {{0x00800000ull, 0x7D000000ull},    // [2^-126, 2^123)
                                         {0x03FE0000ull, 0x7F800000ull},    // [127*2^-126, Inf)
                                         {0x00000000ull, 0x100000000ull},   // every pattern (NaNs skipped)
                                         {0x00000000ull, 0x100000000ull}};  // every pattern

int arith_selfcheck(unsigned long long mismatches[4], hipStream_t stream) {
  const CheckRange *ranges = kRanges;
  unsigned long long *d = nullptr;
  if (hipMalloc(&d, sizeof(unsigned long long) * kCheckBlocks * kChecks) != hipSuccess) return -1;
  for (int w = 0; w < kChecks; ++w)
    enqueue(arith_check_kernel, dim3(kCheckBlocks), dim3(256), 0, stream, w, ranges[w].lo,
                       ranges[w].hi - ranges[w].lo, d + (size_t)w * kCheckBlocks);
  std::vector<unsigned long long> h((size_t)kCheckBlocks * kChecks);
  int rc = 0;
  if (hipGetLastError() != hipSuccess ||
      hipMemcpyAsync(h.data(), d, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost, stream) !=
          hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    rc = -1;
  (void)hipFree(d);
  if (rc) return rc;
  for (int w = 0; w < kChecks; ++w) {
    unsigned long long t = 0;
    for (int b = 0; b < kCheckBlocks; ++b) t += h[(size_t)w * kCheckBlocks + b];
    mismatches[w] = t;
  }
  return 0;
}

// ---------------------------------------------------------------------------
// The non-allocating form: the four counters live in `scratch`, a file-scope
// device array (32 bytes; each device holds its own copy until the process
// ends).  Host code never passes the array's name to a kernel: on the host it
// is a stand-in, not a device address.  The device address comes from
// hipGetSymbolAddress, called once per device with that device current, on the
// entry's first call there.  Every call on a device shares its counters and
// clears them first, so a call holds that device's lock from the clear until
// its counts are back on the host: calls from several host threads on one
// device run one after another instead of racing on the counters.
static __device__ __align__(256) unsigned long long scratch[kChecks];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static unsigned long long *g_scratch_ptr[kMaxDevices];
static std::mutex g_device_mu[kMaxDevices];  // one call at a time per device

// The address of `scratch` on device dev (current), or nullptr on a HIP error.
static unsigned long long *scratch_on_device(int dev) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    g_scratch_ptr[dev] = static_cast<unsigned long long *>(p);
  }
  return g_scratch_ptr[dev];
}

int arith_selfcheck_noalloc(unsigned long long mismatches[4], int checks, hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -1;
  std::lock_guard<std::mutex> call_lock(g_device_mu[dev]);
  unsigned long long *counters = scratch_on_device(dev);
  if (!counters) return -1;
  enqueue(clear_counters_kernel, dim3(1), dim3(64), 0, stream, counters, kChecks);
  for (int w = 0; w < kChecks; ++w)
    if (checks & (1 << w))
      enqueue(arith_count_kernel, dim3(kCheckBlocks), dim3(256), 0, stream, w, kRanges[w].lo,
              kRanges[w].hi - kRanges[w].lo, counters + w);
  unsigned long long h[kChecks] = {0, 0, 0, 0};
  if (hipGetLastError() != hipSuccess ||
      hipMemcpyAsync(h, counters, sizeof(h), hipMemcpyDeviceToHost, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    return -1;
  for (int w = 0; w < kChecks; ++w)
    if (checks & (1 << w)) mismatches[w] = h[w];
  return 0;
}

}  // namespace v7g
