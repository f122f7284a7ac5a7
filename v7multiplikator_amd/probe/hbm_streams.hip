// hbm_streams.hip -- HBM ceilings of plain streaming kernels on one GPU, by
// access mix: the bound each kernel of the library is compared against.
//
//   v7g_hbm_streams [--iterations N]
//
// Every mode streams float4 (16 bytes per lane, one per thread unless stated)
// with nontemporal loads and stores, as the library's kernels do, over arrays
// of 2^25 floats (128 MiB); three buffer sets rotate so that no launch is
// served from the Infinity Cache.  HIP events around N back-to-back launches;
// one JSON line per mode: {"mode", "bytes", "us", "GB/s", "frac"} (frac of 8 TB/s).
//
//   read       x = a[i] (kept live by a never-true compare)         1 read
//   write      c[i] = constant                                      1 write
//   copy       c[i] = a[i]                                          1R 1W
//   inplace    a[i] = 2 a[i]                                        1R 1W, same array
//   inplace8   a[i] = 2 a[i], 8 lanes per 512-byte unit, 4 float4 per lane
//              at a 128-byte stride (the 8-lane RMSNorm+RoPE layout)  1R 1W
//   add        c[i] = a[i] + b[i]                                   2R 1W
//   add_inplace2  x = a[i] + b[i]; a[i] = x; c[i] = 2x              2R 2W (add+RMSNorm's mix)
//   dup        c[i] = a[i]; d[i] = 2 a[i]                           1R 2W
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

__device__ inline f4 ld(const f4 *p) { return __builtin_nontemporal_load(p); }
__device__ inline void st(f4 *p, f4 v) { __builtin_nontemporal_store(v, p); }

enum Mode { READ, WRITE, COPY, INPLACE, INPLACE8, ADD, ADD_INPLACE2, DUP, N_MODES };
const char *kNames[N_MODES] = {"read", "write", "copy", "inplace", "inplace8", "add", "add_inplace2", "dup"};
const int kArrays[N_MODES][2] = {{1, 0}, {0, 1}, {1, 1}, {1, 1}, {1, 1}, {2, 1}, {2, 2}, {1, 2}};  // reads, writes

template <int MODE>
__global__ __launch_bounds__(256) void stream_kernel(f4 *a, const f4 *b, f4 *c, f4 *d, long long n4) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  if constexpr (MODE == READ) {
    const f4 x = ld(a + i);
    if (x.x == 1234.5f && x.y == -1234.5f) c[0] = x;  // never true for the zero-filled input
  } else if constexpr (MODE == WRITE) {
    st(c + i, f4{1.f, 2.f, 3.f, 4.f});
  } else if constexpr (MODE == COPY) {
    st(c + i, ld(a + i));
  } else if constexpr (MODE == INPLACE) {
    st(a + i, ld(a + i) * 2.0f);
  } else if constexpr (MODE == ADD) {
    st(c + i, ld(a + i) + ld(b + i));
  } else if constexpr (MODE == ADD_INPLACE2) {
    const f4 x = ld(a + i) + ld(b + i);
    st(a + i, x);
    st(c + i, x * 2.0f);
  } else if constexpr (MODE == DUP) {
    const f4 x = ld(a + i);
    st(c + i, x);
    st(d + i, x * 2.0f);
  }
}

// Units of 32 float4 (512 bytes), 8 lanes each: lane m holds float4 m + 8k, k < 4.
__global__ __launch_bounds__(256) void inplace8_kernel(f4 *a, long long n4) {
  const long long unit = ((long long)blockIdx.x * 256 + threadIdx.x) >> 3;
  const int m = threadIdx.x & 7;
  if (unit >= n4 / 32) return;
  f4 *p = a + unit * 32 + m;
  f4 x[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) x[k] = ld(p + 8 * k);
#pragma unroll
  for (int k = 0; k < 4; ++k) st(p + 8 * k, x[k] * 2.0f);
}

void launch(int mode, f4 *const *B, long long n4) {
  const unsigned grid = (unsigned)((n4 + 255) / 256);
  switch (mode) {
#define CASE(M) \
  case M: hipLaunchKernelGGL(stream_kernel<M>, dim3(grid), dim3(256), 0, 0, B[0], B[1], B[2], B[3], n4); break;
    CASE(READ) CASE(WRITE) CASE(COPY) CASE(INPLACE) CASE(ADD) CASE(ADD_INPLACE2) CASE(DUP)
#undef CASE
    case INPLACE8:
      hipLaunchKernelGGL(inplace8_kernel, dim3((unsigned)((n4 / 32 * 8 + 255) / 256)), dim3(256), 0, 0, B[0], n4);
      break;
  }
}

}  // namespace

int main(int argc, char **argv) {
  int iterations = 30;
  for (int i = 1; i < argc; ++i)
    if (!strcmp(argv[i], "--iterations") && i + 1 < argc) iterations = atoi(argv[++i]);
  if (iterations < 1) {
    fprintf(stderr, "usage: v7g_hbm_streams [--iterations N]\n");
    return 1;
  }
  const long long n = 1ll << 25, n4 = n / 4;  // n4 % 256 == 0 and n4 % 32 == 0: every grid covers the arrays exactly
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
    for (int w = 0; w < SETS; ++w) launch(mode, buf[w % SETS], n4);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipEventRecord(e0, 0));
    for (int it = 0; it < iterations; ++it) launch(mode, buf[it % SETS], n4);
    CHECK(hipEventRecord(e1, 0));
    CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    const double us = 1e3 * ms / iterations;
    const double bytes = (double)(kArrays[mode][0] + kArrays[mode][1]) * n * sizeof(float);
    printf("{\"mode\": \"%s\", \"bytes\": %.0f, \"us\": %.3f, \"GB/s\": %.1f, \"frac\": %.4f}\n", kNames[mode], bytes, us,
           bytes / us / 1e3, bytes / us / 1e3 / 8000.0);
    fflush(stdout);
  }
  for (auto &set : buf)
    for (auto &p : set) CHECK(hipFree(p));
  return 0;
}
