// hbm_streams.hip -- HBM ceilings of plain streaming kernels on one GPU, the
// bound each kernel of the library is compared against.  A measurement
// program, built on request (build.build_stream_probe()) into
// v7multiplikator_amd/measure/v7g_hbm_streams; it is not part of libv7g.so.
//
//   v7g_hbm_streams [--iterations N]
//
// Arrays of 2^25 floats (128 MiB); three buffer sets rotate so that no launch
// is served from the Infinity Cache.  HIP events around N back-to-back
// launches; one JSON line per mode: {"mode", "bytes", "us", "GB/s", "frac"}
// (frac of 8 TB/s).  Unless a mode says otherwise every lane moves one float4
// with nontemporal loads and stores, the library kernels' form.
//
// Access mixes (the library's kernels are compared with the mix they move):
//   read          x = a[i], kept live by a compare that is never true    1R
//   write         c[i] = constant                                        1W
//   copy          c[i] = a[i]                                            1R 1W
//   inplace       a[i] = 2 a[i]                                          1R 1W, one array
//   inplace8      inplace with 8 lanes per 512-byte unit, 4 float4 per
//                 lane at a 128-byte stride (the RMSNorm+RoPE lane layout) 1R 1W
//   add           c[i] = a[i] + b[i]                                     2R 1W
//   add_inplace2  x = a[i] + b[i]; a[i] = x; c[i] = 2x                   2R 2W (add+RMSNorm)
//   dup           c[i] = a[i]; d[i] = 2 a[i]                             1R 2W
// Load and store forms, against read / write / add above:
//   read_plain, write_plain     ordinary (cached) loads / stores
//   add_plain_ld, add_plain_st  add with ordinary loads / ordinary stores
//   read_x4       4 float4 per lane (block-contiguous, 4 KiB per wave per load)
//   read_buffer   buffer_load_dwordx4 nt (a raw buffer resource over the array)
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

#define CHECK(x)                                                                 \
  do {                                                                           \
    hipError_t e_ = (x);                                                         \
    if (e_ != hipSuccess) {                                                      \
      fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));             \
      exit(1);                                                                   \
    }                                                                            \
  } while (0)

template <bool NT>
__device__ inline f4 ld(const f4 *p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  return *p;
}
template <bool NT>
__device__ inline void st(f4 *p, f4 v) {
  if constexpr (NT)
    __builtin_nontemporal_store(v, p);
  else
    *p = v;
}
// keeps a loaded value live without a store that could ever run (inputs are zero-filled)
__device__ inline void keep(f4 x, f4 *sink) {
  if (x.x == 1234.5f && x.y == -1234.5f) sink[0] = x;
}

enum Mode {
  READ, WRITE, COPY, INPLACE, INPLACE8, ADD, ADD_INPLACE2, DUP,
  READ_PLAIN, WRITE_PLAIN, ADD_PLAIN_LD, ADD_PLAIN_ST, READ_X4, READ_BUFFER, N_MODES
};
const char *kNames[N_MODES] = {"read",       "write",       "copy",         "inplace",      "inplace8",
                               "add",        "add_inplace2", "dup",         "read_plain",   "write_plain",
                               "add_plain_ld", "add_plain_st", "read_x4",   "read_buffer"};
const int kArrays[N_MODES] = {1, 1, 2, 2, 2, 3, 4, 3, 1, 1, 3, 3, 1, 1};  // arrays read + written

// One float4 per lane, grid = n4 / 256 blocks of 256 threads.
template <int MODE>
__global__ __launch_bounds__(256) void stream_kernel(f4 *a, const f4 *b, f4 *c, f4 *d, long long n4) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  if constexpr (MODE == READ) {
    keep(ld<true>(a + i), c);
  } else if constexpr (MODE == READ_PLAIN) {
    keep(ld<false>(a + i), c);
  } else if constexpr (MODE == WRITE) {
    st<true>(c + i, f4{1.f, 2.f, 3.f, 4.f});
  } else if constexpr (MODE == WRITE_PLAIN) {
    st<false>(c + i, f4{1.f, 2.f, 3.f, 4.f});
  } else if constexpr (MODE == COPY) {
    st<true>(c + i, ld<true>(a + i));
  } else if constexpr (MODE == INPLACE) {
    st<true>(a + i, ld<true>(a + i) * 2.0f);
  } else if constexpr (MODE == ADD) {
    st<true>(c + i, ld<true>(a + i) + ld<true>(b + i));
  } else if constexpr (MODE == ADD_PLAIN_LD) {
    st<true>(c + i, ld<false>(a + i) + ld<false>(b + i));
  } else if constexpr (MODE == ADD_PLAIN_ST) {
    st<false>(c + i, ld<true>(a + i) + ld<true>(b + i));
  } else if constexpr (MODE == ADD_INPLACE2) {
    const f4 x = ld<true>(a + i) + ld<true>(b + i);
    st<true>(a + i, x);
    st<true>(c + i, x * 2.0f);
  } else if constexpr (MODE == DUP) {
    const f4 x = ld<true>(a + i);
    st<true>(c + i, x);
    st<true>(d + i, x * 2.0f);
  }
}

// Units of 32 float4 (512 bytes), 8 lanes each: lane m holds float4 m + 8k, k < 4.
__global__ __launch_bounds__(256) void inplace8_kernel(f4 *a, long long n4) {
  const long long unit = ((long long)blockIdx.x * 256 + threadIdx.x) >> 3;
  if (unit >= n4 / 32) return;
  f4 *p = a + unit * 32 + (threadIdx.x & 7);
  f4 x[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) x[k] = ld<true>(p + 8 * k);
#pragma unroll
  for (int k = 0; k < 4; ++k) st<true>(p + 8 * k, x[k] * 2.0f);
}

// Block b covers float4 1024 b .. 1024 b + 1023; lane t loads t + 256 k, k < 4.
__global__ __launch_bounds__(256) void read_x4_kernel(const f4 *a, f4 *sink, long long n4) {
  const long long base = (long long)blockIdx.x * 1024 + threadIdx.x;
  if (base + 768 >= n4) return;
  f4 x[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) x[k] = ld<true>(a + base + 256 * k);
  keep(x[0] + x[1] + x[2] + x[3], sink);
}

// The same walk as read_x4 through a raw buffer resource (byte offsets < 2^31).
__global__ __launch_bounds__(256) void read_buffer_kernel(const f4 *a, f4 *sink, long long n4) {
  const long long base = (long long)blockIdx.x * 1024 + threadIdx.x;
  if (base + 768 >= n4) return;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<f4 *>(a), 0, (int)(n4 * 16 < 0x7fffffff ? n4 * 16 : 0x7fffffff),
                                        0x00020000);
  f4 x[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    x[k] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, (unsigned)(base + 256 * k) * 16u, 0, 2));
  keep(x[0] + x[1] + x[2] + x[3], sink);
}

void launch(int mode, f4 *const *B, long long n4) {
  const unsigned grid = (unsigned)((n4 + 255) / 256);
  switch (mode) {
#define CASE(M) \
  case M: hipLaunchKernelGGL(stream_kernel<M>, dim3(grid), dim3(256), 0, 0, B[0], B[1], B[2], B[3], n4); break;
    CASE(READ) CASE(WRITE) CASE(COPY) CASE(INPLACE) CASE(ADD) CASE(ADD_INPLACE2) CASE(DUP)
    CASE(READ_PLAIN) CASE(WRITE_PLAIN) CASE(ADD_PLAIN_LD) CASE(ADD_PLAIN_ST)
#undef CASE
    case INPLACE8:
      hipLaunchKernelGGL(inplace8_kernel, dim3((unsigned)((n4 / 32 * 8 + 255) / 256)), dim3(256), 0, 0, B[0], n4);
      break;
    case READ_X4:
      hipLaunchKernelGGL(read_x4_kernel, dim3((unsigned)(n4 / 1024)), dim3(256), 0, 0, B[0], B[2], n4);
      break;
    case READ_BUFFER:
      hipLaunchKernelGGL(read_buffer_kernel, dim3((unsigned)(n4 / 1024)), dim3(256), 0, 0, B[0], B[2], n4);
      break;
  }
}

}  // namespace

int main(int argc, char **argv) {
  int iterations = 30;
  bool ok = true;
  for (int i = 1; i < argc; ++i) {
    if (!strcmp(argv[i], "--iterations") && i + 1 < argc)
      iterations = atoi(argv[++i]);
    else
      ok = false;
  }
  if (!ok || iterations < 1) {
    printf("usage: v7g_hbm_streams [--iterations N]\n");
    return 1;
  }
  // n4 is a multiple of 1024: every grid above covers the arrays exactly
  const long long n = 1ll << 25, n4 = n / 4;
  constexpr int SETS = 3;
  f4 *buf[SETS][4];
  for (auto &set : buf)
    for (auto &p : set) {
      CHECK(hipMalloc(&p, n * sizeof(float)));
      CHECK(hipMemset(p, 0, n * sizeof(float)));
    }
  int dev = 0;
  hipDeviceProp_t prop;
  CHECK(hipGetDevice(&dev));
  CHECK(hipGetDeviceProperties(&prop, dev));
  printf("device %d: %s (%s), %d CUs\n", dev, prop.name, prop.gcnArchName, prop.multiProcessorCount);
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  for (int mode = 0; mode < N_MODES; ++mode) {
    for (int w = 0; w < SETS; ++w) launch(mode, buf[w], n4);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipEventRecord(e0, 0));
    for (int it = 0; it < iterations; ++it) launch(mode, buf[it % SETS], n4);
    CHECK(hipEventRecord(e1, 0));
    CHECK(hipEventSynchronize(e1));
    CHECK(hipGetLastError());
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    const double us = 1e3 * ms / iterations;
    const double bytes = (double)kArrays[mode] * n * sizeof(float);
    printf("{\"mode\": \"%s\", \"bytes\": %.0f, \"us\": %.3f, \"GB/s\": %.1f, \"frac\": %.4f}\n", kNames[mode], bytes,
           us, bytes / us / 1e3, bytes / us / 1e3 / 8000.0);
    fflush(stdout);
  }
  for (auto &set : buf)
    for (auto &p : set) CHECK(hipFree(p));
  return 0;
}
