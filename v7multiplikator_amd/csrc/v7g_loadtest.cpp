// v7g_loadtest.cpp -- GPU leg of the reference's kernel load benchmarks
// (tools/b_fused_add_rmsnorm_loadtest.cpp, b_rmsnorm_rope_loadtest.cpp,
// b_swiglu_loadtest.cpp, b_swiglu_q8_loadtest.cpp, and the adjacent
// b_rmsnorm_loadtest.cpp and b_add_inplace_loadtest.cpp): times one kernel of
// libv7g.so on one GPU and prints the reference's "Pass: ... us / call (GB/s)"
// lines, plus the fraction of MI355X's 8 TB/s HBM peak.
//
//   v7g_loadtest <libv7g.so> fused_add_rmsnorm <rows> <dim>
//   v7g_loadtest <libv7g.so> rmsnorm <rows> <dim>           (tools/b_rmsnorm_loadtest.cpp)
//   v7g_loadtest <libv7g.so> add_inplace <rows> <dim>       (tools/b_add_inplace_loadtest.cpp)
//   v7g_loadtest <libv7g.so> rmsnorm_rope <tokens> <q_heads> <kv_heads> <head_dim>
//   v7g_loadtest <libv7g.so> swiglu <rows> <hidden>
//   v7g_loadtest <libv7g.so> swiglu_q8 <rows> <hidden> [gs]
//   v7g_loadtest <libv7g.so> embedding <tokens> <vocab> <dim>
//   v7g_loadtest <libv7g.so> rmsnorm_quantize <rows> <dim> [gs]
//   v7g_loadtest <libv7g.so> add_rmsnorm_quantize <rows> <dim> [gs]
//   v7g_loadtest <libv7g.so> kv_pack <tokens> <kv_dim>       (two launches, one per side)
//   v7g_loadtest <libv7g.so> kv_pack_kv <tokens> <kv_dim>    (K and V in one launch)
//   v7g_loadtest <libv7g.so> qkv_stage <tokens> <q_heads> <kv_heads> <head_dim>
//   v7g_loadtest <libv7g.so> rope_only <tokens> <q_heads> <kv_heads> <head_dim> [bias 0|1]
//   v7g_loadtest <libv7g.so> configs          (every benchmark configuration below)
//   v7g_loadtest <libv7g.so> next             (the widened rows at the Qwen3-8B T=8192 shape)
//   v7g_loadtest <libv7g.so> models [tokens] [name]  (the per-layer kernels at other model shapes)
//   v7g_loadtest <libv7g.so> decode [tokens]  (small-batch steps: eager launches against HIP graphs)
//   options: --iterations N  --time secs  --no-rotate  --per-row
//
// Like the reference harnesses it loads the library with dlopen and resolves
// each entry by name (src/v7_lib.h:585-739), warms up, optionally calibrates
// the iteration count to --time, then times `iterations` calls.  Differences
// that the GPU requires: buffers are device memory (hipMalloc) filled once
// from a seeded host generator; time comes from HIP events on the library
// stream; and, unless --no-rotate, the calls cycle through as many copies of
// the buffers as it takes to exceed 512 MiB, so small shapes are not served
// from the 256 MiB Infinity Cache (a cache-resident number is printed with
// --no-rotate and labelled so).  --per-row calls the reference-signature
// entry once per row, as the reference engine drives its kernels, to show
// what a per-row launch costs on a GPU.  Bytes per call count every tensor
// once (inputs read once, outputs written once).
#include <dlfcn.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <chrono>
#include <thread>
#include <vector>

#include "v7g_lib.h"

namespace {

#define HIPCHECK(x)                                                                        \
  do {                                                                                     \
    hipError_t e_ = (x);                                                                   \
    if (e_ != hipSuccess) {                                                                \
      printf("Fail: HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      exit(1);                                                                             \
    }                                                                                      \
  } while (0)

const double kPeakGBs = 8000.0;

struct Lib {
  void *h = nullptr;
  int (*init)(void);
  void (*set_stream)(void *);
  int (*sync)(void);
  int (*get_last_error)(void);
  const char *(*error_string)(int);
  int (*build_rope_tables)(float *, float *, int, int, float);
  int (*fused_add_rmsnorm)(float *, float *, const float *, const float *, int, int, float);
  int (*rmsnorm)(float *, const float *, const float *, int, int, float);
  int (*add_inplace)(float *, const float *, long long);
  int (*qk_rmsnorm_rope)(float *, long long, int, const float *, float *, long long, int, const float *, int, int,
                         const float *, const float *, const int32_t *, int, int, int, float);
  int (*swiglu_f32)(float *, const float *, const float *, long long);
  int (*swiglu_q8)(int8_t *, float *, const float *, const float *, int, int, int);
  int (*embedding_gather_q8)(float *, const int32_t *, int, const int8_t *, const float *, int, int);
  int (*rmsnorm_quantize)(int8_t *, float *, const float *, const float *, int, int, int, float);
  int (*add_rmsnorm_quantize)(int8_t *, float *, float *, const float *, const float *, int, int, int, float);
  int (*kv_pack_f16)(uint16_t *, long long, const float *, long long, int, int);
  int (*kv_pack_f16_kv)(uint16_t *, long long, uint16_t *, long long, const float *, const float *, long long, int,
                        int);
  int (*qkv_rope_stage)(const v7g_qkv_stage *);
  v7s_fused_add_rmsnorm_fn v7s_fused_add_rmsnorm;
  v7s_rmsnorm_fn v7s_rmsnorm;
  v7s_add_inplace_fn v7s_add_inplace;
  v7s_rmsnorm_rope_heads_fn v7s_rmsnorm_rope_heads;
  v7s_swiglu_quantize_row_fn v7s_swiglu_quantize_row;
  v7s_swiglu_row_fn v7s_swiglu_row;
  v7s_embedding_row_fn v7s_embedding_row;
};

template <typename F>
void resolve(Lib &L, F &fn, const char *name) {
  void *p = dlsym(L.h, name);
  if (!p) {
    printf("[FATAL] missing symbol %s\n", name);
    exit(1);
  }
  memcpy(&fn, &p, sizeof(p));
}

int load(const char *path, Lib &L) {
  L.h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
  if (!L.h) {
    printf("[v7g_loadtest] failed to load %s: %s\n", path, dlerror());
    return -1;
  }
  resolve(L, L.init, "v7g_init");
  resolve(L, L.set_stream, "v7g_set_stream");
  resolve(L, L.sync, "v7g_sync");
  resolve(L, L.get_last_error, "v7g_get_last_error");
  resolve(L, L.error_string, "v7g_error_string");
  resolve(L, L.build_rope_tables, "v7g_build_rope_tables");
  resolve(L, L.fused_add_rmsnorm, "v7g_fused_add_rmsnorm");
  resolve(L, L.rmsnorm, "v7g_rmsnorm");
  resolve(L, L.add_inplace, "v7g_add_inplace");
  resolve(L, L.qk_rmsnorm_rope, "v7g_qk_rmsnorm_rope");
  resolve(L, L.swiglu_f32, "v7g_swiglu_f32");
  resolve(L, L.swiglu_q8, "v7g_swiglu_q8");
  resolve(L, L.embedding_gather_q8, "v7g_embedding_gather_q8");
  resolve(L, L.rmsnorm_quantize, "v7g_rmsnorm_quantize");
  resolve(L, L.add_rmsnorm_quantize, "v7g_add_rmsnorm_quantize");
  resolve(L, L.kv_pack_f16, "v7g_kv_pack_f16");
  resolve(L, L.kv_pack_f16_kv, "v7g_kv_pack_f16_kv");
  resolve(L, L.qkv_rope_stage, "v7g_qkv_rope_stage");
  resolve(L, L.v7s_fused_add_rmsnorm, "v7s_fused_add_rmsnorm");
  resolve(L, L.v7s_rmsnorm, "v7s_rmsnorm");
  resolve(L, L.v7s_add_inplace, "v7s_add_inplace");
  resolve(L, L.v7s_rmsnorm_rope_heads, "v7s_rmsnorm_rope_heads");
  resolve(L, L.v7s_swiglu_quantize_row, "v7s_swiglu_quantize_row");
  resolve(L, L.v7s_swiglu_row, "v7s_swiglu_row");
  resolve(L, L.v7s_embedding_row, "v7s_embedding_row");
  return 0;
}

// splitmix64 -> uniform floats; the shapes, not the values, set the timing.
struct Rng {
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed) {}
  uint64_t next() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  float uniform(float lo, float hi) { return lo + (hi - lo) * (float)((next() >> 40) * (1.0 / 16777216.0)); }
};

template <typename T>
T *device_fill(size_t n, Rng &r, float lo, float hi) {
  std::vector<T> h(n);
  for (size_t i = 0; i < n; ++i) h[i] = (T)r.uniform(lo, hi);
  T *d = nullptr;
  HIPCHECK(hipMalloc(&d, n * sizeof(T)));
  HIPCHECK(hipMemcpy(d, h.data(), n * sizeof(T), hipMemcpyHostToDevice));
  return d;
}

template <typename T>
T *device_empty(size_t n) {
  T *d = nullptr;
  HIPCHECK(hipMalloc(&d, n * sizeof(T)));
  return d;
}

struct Opts {
  int iterations = 200;
  double seconds = 0.0;
  bool rotate = true;
  bool per_row = false;
};

// Number of buffer sets so that one pass over them exceeds 512 MiB.
int sets_for(double bytes_per_call, bool rotate) {
  if (!rotate) return 1;
  int n = (int)((512.0 * 1024 * 1024) / bytes_per_call) + 1;
  return n < 1 ? 1 : (n > 64 ? 64 : n);
}

// Times `call(set)` with HIP events on `stream`: 3 warm-up rounds over every
// set, optional calibration to opt.seconds, then the timed iterations.
template <typename Call>
double time_calls(const Lib &L, hipStream_t stream, int sets, const Opts &opt, Call call, int *iters_out) {
  for (int w = 0; w < 3; ++w)
    for (int s = 0; s < sets; ++s) call(s);
  HIPCHECK(hipStreamSynchronize(stream));
  hipEvent_t a, b;
  HIPCHECK(hipEventCreate(&a));
  HIPCHECK(hipEventCreate(&b));
  int iters = opt.iterations;
  if (opt.seconds > 0.0) {
    HIPCHECK(hipEventRecord(a, stream));
    for (int i = 0; i < 20; ++i) call(i % sets);
    HIPCHECK(hipEventRecord(b, stream));
    HIPCHECK(hipEventSynchronize(b));
    float ms = 0.f;
    HIPCHECK(hipEventElapsedTime(&ms, a, b));
    iters = (int)(opt.seconds * 1e3 / (ms / 20.0) * 0.95);
    if (iters < 10) iters = 10;
  }
  HIPCHECK(hipEventRecord(a, stream));
  for (int i = 0; i < iters; ++i) call(i % sets);
  HIPCHECK(hipEventRecord(b, stream));
  HIPCHECK(hipEventSynchronize(b));
  float ms = 0.f;
  HIPCHECK(hipEventElapsedTime(&ms, a, b));
  HIPCHECK(hipEventDestroy(a));
  HIPCHECK(hipEventDestroy(b));
  int err = L.get_last_error();
  if (err) {
    printf("Fail: library error %d (%s)\n", err, L.error_string(err));
    exit(1);
  }
  *iters_out = iters;
  return ms * 1e3 / iters;  // us per call
}

void report(const char *what, const std::string &shape, int iters, double us, double bytes, int sets) {
  double gbs = bytes / (us * 1e-6) / 1e9;
  const bool resident = bytes * sets < 512.0 * 1024 * 1024;  // the rotation fits the 256 MiB MALL twice over
  printf("Pass: %s %s iterations=%d%s\n", what, shape.c_str(), iters,
         resident ? "  (cache-resident: working set below 512 MiB)" : "");
  printf("  %.3f us / call   (%.1f GB/s, %.1f%% of 8 TB/s)   bytes/call=%.0f buffer_sets=%d\n", us, gbs,
         100.0 * gbs / kPeakGBs, bytes, sets);
  printf("{\"kernel\": \"%s\", \"shape\": \"%s\", \"us\": %.3f, \"GBs\": %.1f, \"frac\": %.4f, \"bytes\": %.0f, "
         "\"buffer_sets\": %d, \"iterations\": %d}\n",
         what, shape.c_str(), us, gbs, gbs / kPeakGBs, bytes, sets, iters);
  fflush(stdout);
}

void run_add_rmsnorm(const Lib &L, hipStream_t st, int rows, int dim, const Opts &opt) {
  const size_t n = (size_t)rows * dim;
  const double bytes = 4.0 * n * 4 + dim * 4.0;
  const int sets = sets_for(bytes, opt.rotate);
  Rng r(1);
  std::vector<float *> res(sets), add(sets), out(sets);
  for (int s = 0; s < sets; ++s) {
    res[s] = device_fill<float>(n, r, -1.f, 1.f);
    add[s] = device_fill<float>(n, r, -1.f, 1.f);
    out[s] = device_empty<float>(n);
  }
  float *w = device_fill<float>(dim, r, 0.5f, 1.5f);
  int iters = 0;
  double us;
  char shape[96];
  if (opt.per_row) {
    us = time_calls(L, st, sets, opt, [&](int s) {
      for (int i = 0; i < rows; ++i)
        L.v7s_fused_add_rmsnorm(out[s] + (size_t)i * dim, res[s] + (size_t)i * dim, add[s] + (size_t)i * dim, w, dim);
    }, &iters);
    snprintf(shape, sizeof shape, "rows=%d dim=%d per-row-calls", rows, dim);
  } else {
    us = time_calls(L, st, sets, opt, [&](int s) { L.fused_add_rmsnorm(out[s], res[s], add[s], w, rows, dim, 1e-6f); },
                    &iters);
    snprintf(shape, sizeof shape, "rows=%d dim=%d", rows, dim);
  }
  report("fused_add_rmsnorm", shape, iters, us, bytes, sets);
  for (int s = 0; s < sets; ++s) {
    HIPCHECK(hipFree(res[s]));
    HIPCHECK(hipFree(add[s]));
    HIPCHECK(hipFree(out[s]));
  }
  HIPCHECK(hipFree(w));
}

// v7s_rmsnorm over rows of dim floats (the reference's b_rmsnorm_loadtest runs one row of `size`): x read,
// o written, the weight once.
void run_rmsnorm(const Lib &L, hipStream_t st, int rows, int dim, const Opts &opt) {
  const size_t n = (size_t)rows * dim;
  const double bytes = 2.0 * n * 4 + dim * 4.0;
  const int sets = sets_for(bytes, opt.rotate);
  Rng r(7);
  std::vector<float *> x(sets), out(sets);
  for (int s = 0; s < sets; ++s) {
    x[s] = device_fill<float>(n, r, -1.f, 1.f);
    out[s] = device_empty<float>(n);
  }
  float *w = device_fill<float>(dim, r, 0.5f, 1.5f);
  int iters = 0;
  double us;
  char shape[96];
  if (opt.per_row) {
    us = time_calls(L, st, sets, opt, [&](int s) {
      for (int i = 0; i < rows; ++i) L.v7s_rmsnorm(out[s] + (size_t)i * dim, x[s] + (size_t)i * dim, w, dim);
    }, &iters);
    snprintf(shape, sizeof shape, "rows=%d dim=%d per-row-calls", rows, dim);
  } else {
    us = time_calls(L, st, sets, opt, [&](int s) { L.rmsnorm(out[s], x[s], w, rows, dim, 1e-6f); }, &iters);
    snprintf(shape, sizeof shape, "rows=%d dim=%d", rows, dim);
  }
  report("rmsnorm", shape, iters, us, bytes, sets);
  for (int s = 0; s < sets; ++s) {
    HIPCHECK(hipFree(x[s]));
    HIPCHECK(hipFree(out[s]));
  }
  HIPCHECK(hipFree(w));
}

// v7s_add_inplace, x += y over rows x dim floats (b_add_inplace_loadtest: one call over n floats): x and y
// read, x written.  Each call adds y once more to its set's x; the values stay finite over any run here.
void run_add_inplace(const Lib &L, hipStream_t st, int rows, int dim, const Opts &opt) {
  const size_t n = (size_t)rows * dim;
  const double bytes = 3.0 * n * 4;
  const int sets = sets_for(bytes, opt.rotate);
  Rng r(8);
  std::vector<float *> x(sets), y(sets);
  for (int s = 0; s < sets; ++s) {
    x[s] = device_fill<float>(n, r, -1.f, 1.f);
    y[s] = device_fill<float>(n, r, -1e-3f, 1e-3f);
  }
  int iters = 0;
  double us;
  char shape[96];
  if (opt.per_row) {
    us = time_calls(L, st, sets, opt, [&](int s) {
      for (int i = 0; i < rows; ++i) L.v7s_add_inplace(x[s] + (size_t)i * dim, y[s] + (size_t)i * dim, dim);
    }, &iters);
    snprintf(shape, sizeof shape, "rows=%d dim=%d per-row-calls", rows, dim);
  } else {
    us = time_calls(L, st, sets, opt, [&](int s) { L.add_inplace(x[s], y[s], (long long)n); }, &iters);
    snprintf(shape, sizeof shape, "rows=%d dim=%d", rows, dim);
  }
  report("add_inplace", shape, iters, us, bytes, sets);
  for (int s = 0; s < sets; ++s) {
    HIPCHECK(hipFree(x[s]));
    HIPCHECK(hipFree(y[s]));
  }
}

void run_rope(const Lib &L, hipStream_t st, int T, int nq, int nk, int hd, const Opts &opt) {
  const long long ts = (long long)(nq + 2 * nk) * hd;  // fused QKV row: [Q | K | V]
  const size_t n = (size_t)T * ts;
  const double bytes = 2.0 * T * (nq + nk) * hd * 4 + 2.0 * T * (hd / 2) * 4 + 2.0 * hd * 4;
  const int sets = sets_for(bytes, opt.rotate);
  Rng r(2);
  std::vector<float *> qkv(sets);
  for (int s = 0; s < sets; ++s) qkv[s] = device_fill<float>(n, r, -1.f, 1.f);
  float *qw = device_fill<float>(hd, r, 0.5f, 1.5f), *kw = device_fill<float>(hd, r, 0.5f, 1.5f);
  float *ct = device_empty<float>((size_t)T * hd / 2), *stb = device_empty<float>((size_t)T * hd / 2);
  if (L.build_rope_tables(ct, stb, T, hd, 1e6f)) {
    printf("Fail: rope tables\n");
    exit(1);
  }
  std::vector<int32_t> hp(T);
  for (int i = 0; i < T; ++i) hp[i] = i;
  int32_t *pos = device_empty<int32_t>(T);
  HIPCHECK(hipMemcpy(pos, hp.data(), T * 4, hipMemcpyHostToDevice));
  int iters = 0;
  double us;
  char shape[128];
  if (opt.per_row) {
    us = time_calls(L, st, sets, opt, [&](int s) {
      for (int t = 0; t < T; ++t) {
        float *row = qkv[s] + (size_t)t * ts;
        L.v7s_rmsnorm_rope_heads(row, nq, hd, qw, ct, stb, t, hd / 2);
        L.v7s_rmsnorm_rope_heads(row + (size_t)nq * hd, nk, hd, kw, ct, stb, t, hd / 2);
      }
    }, &iters);
    snprintf(shape, sizeof shape, "tokens=%d q_heads=%d kv_heads=%d head_dim=%d per-token-calls", T, nq, nk, hd);
  } else {
    us = time_calls(L, st, sets, opt, [&](int s) {
      L.qk_rmsnorm_rope(qkv[s], ts, nq, qw, qkv[s] + (size_t)nq * hd, ts, nk, kw, T, hd, ct, stb, pos, 0, hd / 2, T,
                        1e-6f);
    }, &iters);
    snprintf(shape, sizeof shape, "tokens=%d q_heads=%d kv_heads=%d head_dim=%d", T, nq, nk, hd);
  }
  report("rmsnorm_rope", shape, iters, us, bytes, sets);
  for (int s = 0; s < sets; ++s) HIPCHECK(hipFree(qkv[s]));
  HIPCHECK(hipFree(qw));
  HIPCHECK(hipFree(kw));
  HIPCHECK(hipFree(ct));
  HIPCHECK(hipFree(stb));
  HIPCHECK(hipFree(pos));
}

void run_swiglu(const Lib &L, hipStream_t st, int rows, int hidden, int gs, bool q8, const Opts &opt) {
  const size_t n = (size_t)rows * hidden;
  const double bytes = q8 ? 2.0 * n * 4 + n + (double)rows * (hidden / gs) * 4 : 3.0 * n * 4;
  const int sets = sets_for(bytes, opt.rotate);
  Rng r(3);
  std::vector<float *> g(sets), u(sets), o(sets), sc(sets);
  std::vector<int8_t *> q(sets);
  for (int s = 0; s < sets; ++s) {
    g[s] = device_fill<float>(n, r, -3.f, 3.f);
    u[s] = device_fill<float>(n, r, -3.f, 3.f);
    o[s] = q8 ? nullptr : device_empty<float>(n);
    q[s] = q8 ? device_empty<int8_t>(n) : nullptr;
    sc[s] = q8 ? device_empty<float>((size_t)rows * ((hidden + gs - 1) / gs)) : nullptr;
  }
  int iters = 0;
  double us;
  char shape[96];
  if (opt.per_row) {
    us = time_calls(L, st, sets, opt, [&](int s) {
      for (int i = 0; i < rows; ++i) {
        const size_t off = (size_t)i * hidden;
        if (q8)
          L.v7s_swiglu_quantize_row(reinterpret_cast<char *>(q[s] + off), g[s] + off, u[s] + off,
                                    sc[s] + (size_t)i * ((hidden + 63) / 64), hidden);
        else
          L.v7s_swiglu_row(g[s] + off, u[s] + off, hidden);
      }
    }, &iters);
    snprintf(shape, sizeof shape, "rows=%d hidden=%d%s per-row-calls", rows, hidden, q8 ? " gs=64" : "");
  } else {
    us = time_calls(L, st, sets, opt, [&](int s) {
      if (q8)
        L.swiglu_q8(q[s], sc[s], g[s], u[s], rows, hidden, gs);
      else
        L.swiglu_f32(o[s], g[s], u[s], (long long)n);
    }, &iters);
    if (q8)
      snprintf(shape, sizeof shape, "rows=%d hidden=%d gs=%d", rows, hidden, gs);
    else
      snprintf(shape, sizeof shape, "rows=%d hidden=%d", rows, hidden);
  }
  report(q8 ? "swiglu_q8" : "swiglu_f32", shape, iters, us, bytes, sets);
  for (int s = 0; s < sets; ++s) {
    HIPCHECK(hipFree(g[s]));
    HIPCHECK(hipFree(u[s]));
    if (o[s]) HIPCHECK(hipFree(o[s]));
    if (q[s]) HIPCHECK(hipFree(q[s]));
    if (sc[s]) HIPCHECK(hipFree(sc[s]));
  }
}

void run_embedding(const Lib &L, hipStream_t st, int T, int vocab, int dim, const Opts &opt) {
  const double bytes = (double)T * 4 + (double)T * dim + (double)T * (dim / 64) * 4 + (double)T * dim * 4;
  // The id sets rotate on their own, enough of them that the table rows they touch exceed 512 MiB
  // (the outputs rotate through `sets` buffers as for the other kernels).
  const int sets = sets_for(bytes, opt.rotate);
  const int id_sets = opt.rotate ? sets_for((double)T * dim * (1.0 + 1.0 / 16), true) : 1;
  Rng r(4);
  int8_t *tq = device_empty<int8_t>((size_t)vocab * dim);
  {
    std::vector<int8_t> h((size_t)vocab * dim);
    for (auto &v : h) v = (int8_t)((int)(r.next() % 255u) - 127);
    HIPCHECK(hipMemcpy(tq, h.data(), h.size(), hipMemcpyHostToDevice));
  }
  float *tsc = device_fill<float>((size_t)vocab * dim / 64, r, 0.001f, 0.02f);
  std::vector<int32_t *> ids(id_sets);
  std::vector<float *> out(sets);
  std::vector<std::vector<int32_t>> hids(id_sets, std::vector<int32_t>(T));
  for (int s = 0; s < id_sets; ++s) {
    for (auto &v : hids[s]) v = (int32_t)(r.next() % (uint64_t)vocab);
    ids[s] = device_empty<int32_t>(T);
    HIPCHECK(hipMemcpy(ids[s], hids[s].data(), T * 4, hipMemcpyHostToDevice));
  }
  for (int s = 0; s < sets; ++s) out[s] = device_empty<float>((size_t)T * dim);
  const int cycle = sets * id_sets;  // every (output, id) pairing in turn
  v7g_q8_tensor desc{reinterpret_cast<char *>(tq), tsc};
  int iters = 0;
  double us;
  char shape[96];
  if (opt.per_row) {
    us = time_calls(L, st, cycle, opt, [&](int s) {
      for (int t = 0; t < T; ++t) L.v7s_embedding_row(out[s % sets] + (size_t)t * dim, hids[s / sets][t], dim, &desc);
    }, &iters);
    snprintf(shape, sizeof shape, "tokens=%d vocab=%d dim=%d per-token-calls", T, vocab, dim);
  } else {
    us = time_calls(L, st, cycle, opt, [&](int s) {
      L.embedding_gather_q8(out[s % sets], ids[s / sets], T, tq, tsc, dim, vocab);
    }, &iters);
    snprintf(shape, sizeof shape, "tokens=%d vocab=%d dim=%d", T, vocab, dim);
  }
  report("embedding_gather_q8", shape, iters, us, bytes, sets);
  for (int s = 0; s < id_sets; ++s) HIPCHECK(hipFree(ids[s]));
  for (int s = 0; s < sets; ++s) HIPCHECK(hipFree(out[s]));
  HIPCHECK(hipFree(tq));
  HIPCHECK(hipFree(tsc));
}

void run_norm_q8(const Lib &L, hipStream_t st, int rows, int dim, int gs, bool add_first, const Opts &opt) {
  const size_t n = (size_t)rows * dim;
  const double scales = (double)rows * (dim / gs) * 4;
  const double bytes = add_first ? 2.0 * n * 4 + n * 4.0 + n + scales + dim * 4.0 : n * 4.0 + n + scales + dim * 4.0;
  const int sets = sets_for(bytes, opt.rotate);
  Rng r(5);
  std::vector<float *> x(sets), a(sets), sc(sets);
  std::vector<int8_t *> q(sets);
  for (int s = 0; s < sets; ++s) {
    x[s] = device_fill<float>(n, r, -1.f, 1.f);
    a[s] = add_first ? device_fill<float>(n, r, -1.f, 1.f) : nullptr;
    q[s] = device_empty<int8_t>(n);
    sc[s] = device_empty<float>((size_t)rows * (dim / gs));
  }
  float *w = device_fill<float>(dim, r, 0.5f, 1.5f);
  int iters = 0;
  const double us = time_calls(L, st, sets, opt, [&](int s) {
    if (add_first)
      L.add_rmsnorm_quantize(q[s], sc[s], x[s], a[s], w, rows, dim, gs, 1e-6f);
    else
      L.rmsnorm_quantize(q[s], sc[s], x[s], w, rows, dim, gs, 1e-6f);
  }, &iters);
  char shape[96];
  snprintf(shape, sizeof shape, "rows=%d dim=%d gs=%d", rows, dim, gs);
  report(add_first ? "add_rmsnorm_quantize" : "rmsnorm_quantize", shape, iters, us, bytes, sets);
  for (int s = 0; s < sets; ++s) {
    HIPCHECK(hipFree(x[s]));
    if (a[s]) HIPCHECK(hipFree(a[s]));
    HIPCHECK(hipFree(q[s]));
    HIPCHECK(hipFree(sc[s]));
  }
  HIPCHECK(hipFree(w));
}

// K and V rows of a fused QKV row packed to two binary16 cache buffers: two
// v7g_kv_pack_f16 launches (one per side), or one v7g_kv_pack_f16_kv launch.
void run_kv_pack(const Lib &L, hipStream_t st, int T, int kv_dim, bool one_launch, const Opts &opt) {
  const long long ts = 6LL * kv_dim;  // a QKV row of Qwen3-8B shape: Q = 4 kv_dim, K, V
  const double bytes = 2.0 * T * kv_dim * 4 + 2.0 * T * kv_dim * 2;
  const int sets = sets_for(bytes, opt.rotate);
  Rng r(6);
  std::vector<float *> qkv(sets);
  std::vector<uint16_t *> kc(sets), vc(sets);
  for (int s = 0; s < sets; ++s) {
    qkv[s] = device_fill<float>((size_t)T * ts, r, -2.f, 2.f);
    kc[s] = device_empty<uint16_t>((size_t)T * kv_dim);
    vc[s] = device_empty<uint16_t>((size_t)T * kv_dim);
  }
  int iters = 0;
  const double us = time_calls(L, st, sets, opt, [&](int s) {
    if (one_launch) {
      L.kv_pack_f16_kv(kc[s], kv_dim, vc[s], kv_dim, qkv[s] + 4LL * kv_dim, qkv[s] + 5LL * kv_dim, ts, T, kv_dim);
    } else {
      L.kv_pack_f16(kc[s], kv_dim, qkv[s] + 4LL * kv_dim, ts, T, kv_dim);
      L.kv_pack_f16(vc[s], kv_dim, qkv[s] + 5LL * kv_dim, ts, T, kv_dim);
    }
  }, &iters);
  char shape[96];
  snprintf(shape, sizeof shape, "tokens=%d kv_dim=%d (K and V, %s)", T, kv_dim,
           one_launch ? "one launch" : "two launches");
  report(one_launch ? "kv_pack_f16_kv" : "kv_pack_f16", shape, iters, us, bytes, sets);
  for (int s = 0; s < sets; ++s) {
    HIPCHECK(hipFree(qkv[s]));
    HIPCHECK(hipFree(kc[s]));
    HIPCHECK(hipFree(vc[s]));
  }
}

// The per-token Q/K/V stage of the prefill in one launch: Q/K RMSNorm+RoPE,
// K and V binary16 cache rows, f32 Q kept (K and V f32 not written back).
void run_qkv_stage(const Lib &L, hipStream_t st, int T, int nq, int nk, int hd, const Opts &opt) {
  const long long ts = (long long)(nq + 2 * nk) * hd;
  const double bytes = (double)T * (nq + 2 * nk) * hd * 4 + (double)T * nq * hd * 4 + 2.0 * T * nk * hd * 2 +
                       2.0 * T * (hd / 2) * 4 + 2.0 * hd * 4;
  const int sets = sets_for(bytes, opt.rotate);
  Rng r(7);
  std::vector<float *> qkv(sets);
  std::vector<uint16_t *> kc(sets), vc(sets);
  for (int s = 0; s < sets; ++s) {
    qkv[s] = device_fill<float>((size_t)T * ts, r, -1.f, 1.f);
    kc[s] = device_empty<uint16_t>((size_t)T * nk * hd);
    vc[s] = device_empty<uint16_t>((size_t)T * nk * hd);
  }
  float *qw = device_fill<float>(hd, r, 0.5f, 1.5f), *kw = device_fill<float>(hd, r, 0.5f, 1.5f);
  float *ct = device_empty<float>((size_t)T * hd / 2), *stb = device_empty<float>((size_t)T * hd / 2);
  if (L.build_rope_tables(ct, stb, T, hd, 1e6f)) {
    printf("Fail: rope tables\n");
    exit(1);
  }
  int iters = 0;
  const double us = time_calls(L, st, sets, opt, [&](int s) {
    v7g_qkv_stage g;
    memset(&g, 0, sizeof(g));
    g.q = {qkv[s], ts, nq, qw, nullptr, nullptr, 0, 1};
    g.k = {qkv[s] + (size_t)nq * hd, ts, nk, kw, nullptr, kc[s], (long long)nk * hd, 0};
    g.v = {qkv[s] + (size_t)(nq + nk) * hd, ts, nk, nullptr, nullptr, vc[s], (long long)nk * hd, 0};
    g.n_tokens = T;
    g.head_dim = hd;
    g.cos_table = ct;
    g.sin_table = stb;
    g.positions = nullptr;
    g.pos0 = 0;
    g.rope_max_dim = hd / 2;
    g.table_rows = T;
    g.eps = 1e-6f;
    L.qkv_rope_stage(&g);
  }, &iters);
  char shape[128];
  snprintf(shape, sizeof shape, "tokens=%d q_heads=%d kv_heads=%d head_dim=%d (Q f32, K/V to f16 cache)", T, nq, nk,
           hd);
  report("qkv_rope_stage", shape, iters, us, bytes, sets);
  for (int s = 0; s < sets; ++s) {
    HIPCHECK(hipFree(qkv[s]));
    HIPCHECK(hipFree(kc[s]));
    HIPCHECK(hipFree(vc[s]));
  }
  HIPCHECK(hipFree(qw));
  HIPCHECK(hipFree(kw));
  HIPCHECK(hipFree(ct));
  HIPCHECK(hipFree(stb));
}

// The Q/K step of a model without per-head norms, in place inside the fused
// QKV row: RoPE only on Q and K, and with `bias` the QKV bias added to Q, K
// and V first (src/asm/prefill_q8.inc:848-883 without the cache stores).
void run_rope_only(const Lib &L, hipStream_t st, int T, int nq, int nk, int hd, bool bias, const Opts &opt) {
  const long long ts = (long long)(nq + 2 * nk) * hd;
  const int rw = nq + nk + (bias ? nk : 0);  // heads read and written per token
  const double bytes = 2.0 * T * rw * hd * 4 + 2.0 * T * (hd / 2) * 4 + (bias ? (nq + 2.0 * nk) * hd * 4 : 0.0);
  const int sets = sets_for(bytes, opt.rotate);
  Rng r(8);
  std::vector<float *> qkv(sets);
  for (int s = 0; s < sets; ++s) qkv[s] = device_fill<float>((size_t)T * ts, r, -1.f, 1.f);
  float *b = bias ? device_fill<float>((size_t)ts, r, -0.5f, 0.5f) : nullptr;
  float *ct = device_empty<float>((size_t)T * hd / 2), *stb = device_empty<float>((size_t)T * hd / 2);
  if (L.build_rope_tables(ct, stb, T, hd, 1e6f)) {
    printf("Fail: rope tables\n");
    exit(1);
  }
  int iters = 0;
  const double us = time_calls(L, st, sets, opt, [&](int s) {
    v7g_qkv_stage g;
    memset(&g, 0, sizeof(g));
    g.q = {qkv[s], ts, nq, nullptr, b, nullptr, 0, 1};
    g.k = {qkv[s] + (size_t)nq * hd, ts, nk, nullptr, b ? b + (size_t)nq * hd : nullptr, nullptr, 0, 1};
    if (bias) g.v = {qkv[s] + (size_t)(nq + nk) * hd, ts, nk, nullptr, b + (size_t)(nq + nk) * hd, nullptr, 0, 1};
    g.n_tokens = T;
    g.head_dim = hd;
    g.cos_table = ct;
    g.sin_table = stb;
    g.rope_max_dim = hd / 2;
    g.table_rows = T;
    g.eps = 1e-6f;
    L.qkv_rope_stage(&g);
  }, &iters);
  char shape[128];
  snprintf(shape, sizeof shape, "tokens=%d q_heads=%d kv_heads=%d head_dim=%d (RoPE only%s)", T, nq, nk, hd,
           bias ? ", QKV bias" : "");
  report("qkv_rope_stage", shape, iters, us, bytes, sets);
  for (int s = 0; s < sets; ++s) HIPCHECK(hipFree(qkv[s]));
  if (b) HIPCHECK(hipFree(b));
  HIPCHECK(hipFree(ct));
  HIPCHECK(hipFree(stb));
}

// Open-weight model shapes (widths within the dim % 64, hidden % 64 and head_dim % 32 in [64, 512] contract of
// tools/db_build_tool.c:2283-2300) for the `models` mode.
struct ModelShape {
  const char *name;
  int dim, nq, nkv, hd, hidden, vocab;
  bool qk_norm, qkv_bias;
};

const ModelShape kModels[] = {
    {"Qwen2.5-0.5B", 896, 14, 2, 64, 4864, 151936, false, true},
    {"Qwen3-0.6B", 1024, 16, 8, 128, 3072, 151936, true, false},
    {"Gemma-3-1B", 1152, 4, 1, 256, 6912, 262144, true, false},
    {"Llama-3.2-1B", 2048, 32, 8, 64, 8192, 128256, false, false},
    {"TinyLlama-1.1B", 2048, 32, 4, 64, 5632, 32000, false, false},
    {"Qwen2.5-1.5B", 1536, 12, 2, 128, 8960, 151936, false, true},
    {"Gemma-2-2B", 2304, 8, 4, 256, 9216, 256000, false, false},
    {"Qwen3-4B", 2560, 32, 8, 128, 9728, 151936, true, false},
    {"Phi-3-mini", 3072, 32, 32, 96, 8192, 32064, false, false},
    {"Qwen2.5-7B", 3584, 28, 4, 128, 18944, 152064, false, true},
    {"Gemma-3-12B", 3840, 16, 8, 256, 15360, 262144, true, false},
    {"Llama-3-8B", 4096, 32, 8, 128, 14336, 128256, false, false},
    {"Qwen3-14B", 5120, 40, 8, 128, 17408, 151936, true, false},
    {"Llama-3-70B", 8192, 64, 8, 128, 28672, 128256, false, false},
};

// The four per-layer kernels of each model in kModels over `tokens` tokens.
void run_models(const Lib &L, hipStream_t st, int tokens, const char *only, const Opts &opt) {
  for (const ModelShape &m : kModels) {
    if (only && strcmp(only, m.name)) continue;
    printf("== %s: dim %d, %d Q / %d KV heads of %d, hidden %d, vocab %d%s%s\n", m.name, m.dim, m.nq, m.nkv, m.hd,
           m.hidden, m.vocab, m.qk_norm ? ", Q/K norm" : "", m.qkv_bias ? ", QKV bias" : "");
    fflush(stdout);
    run_embedding(L, st, tokens, m.vocab, m.dim, opt);
    run_add_rmsnorm(L, st, tokens, m.dim, opt);
    if (m.qk_norm)
      run_rope(L, st, tokens, m.nq, m.nkv, m.hd, opt);
    else
      run_rope_only(L, st, tokens, m.nq, m.nkv, m.hd, m.qkv_bias, opt);
    run_swiglu(L, st, tokens, m.hidden, 32, true, opt);
  }
}

// Small-batch (decode) steps at the Qwen3-8B shape: per step the embedding gather, add+RMSNorm, the Q/K/V
// stage (Q/K RMSNorm+RoPE, K and V to their binary16 cache rows, one launch) and SwiGLU -> Q8 for `tokens`
// tokens.  Eager launches (host time per call and step time), one HIP graph per step replayed, and one graph
// of all the steps.
void run_decode(const Lib &L, hipStream_t st, int T, const Opts &opt) {
  const int DIM = 4096, VOCAB = 151936, NQ = 32, NKV = 8, HD = 128, HID = 12288, GS = 32, POS = 4096;
  const int N = opt.iterations;
  const long long qs = (long long)(NQ + 2 * NKV) * HD;
  Rng r(9);
  int8_t *tq = device_empty<int8_t>((size_t)VOCAB * DIM);
  HIPCHECK(hipMemset(tq, 1, (size_t)VOCAB * DIM));
  float *ts = device_fill<float>((size_t)VOCAB * DIM / 64, r, 0.001f, 0.02f);
  float *out = device_empty<float>((size_t)T * DIM), *normed = device_empty<float>((size_t)T * DIM);
  float *res = device_fill<float>((size_t)T * DIM, r, -1.f, 1.f), *w = device_fill<float>(DIM, r, 0.5f, 1.5f);
  float *qkv = device_fill<float>((size_t)T * qs, r, -1.f, 1.f);
  float *qw = device_fill<float>(HD, r, 0.5f, 1.5f), *kw = device_fill<float>(HD, r, 0.5f, 1.5f);
  float *gate = device_fill<float>((size_t)T * HID, r, -3.f, 3.f), *up = device_fill<float>((size_t)T * HID, r, -3.f, 3.f);
  int8_t *codes = device_empty<int8_t>((size_t)T * HID);
  float *scales = device_empty<float>((size_t)T * HID / GS);
  uint16_t *kc = device_empty<uint16_t>((size_t)T * NKV * HD), *vc = device_empty<uint16_t>((size_t)T * NKV * HD);
  float *ct = device_empty<float>((size_t)POS * HD / 2), *stb = device_empty<float>((size_t)POS * HD / 2);
  if (L.build_rope_tables(ct, stb, POS, HD, 1e6f)) {
    printf("Fail: rope tables\n");
    exit(1);
  }
  std::vector<int32_t> hv(T);
  for (int i = 0; i < T; ++i) hv[i] = (int32_t)(((uint64_t)i * 7919u) % VOCAB);
  int32_t *ids = device_empty<int32_t>(T), *pos = device_empty<int32_t>(T);
  HIPCHECK(hipMemcpy(ids, hv.data(), T * 4, hipMemcpyHostToDevice));
  for (int i = 0; i < T; ++i) hv[i] = (1000 + i) % POS;
  HIPCHECK(hipMemcpy(pos, hv.data(), T * 4, hipMemcpyHostToDevice));
  int bad = 0;
  auto step = [&]() {
    bad |= L.embedding_gather_q8(out, ids, T, tq, ts, DIM, VOCAB);
    bad |= L.fused_add_rmsnorm(normed, res, out, w, T, DIM, 1e-6f);
    v7g_qkv_stage g;
    memset(&g, 0, sizeof(g));
    g.q = {qkv, qs, NQ, qw, nullptr, nullptr, 0, 1};
    g.k = {qkv + NQ * HD, qs, NKV, kw, nullptr, kc, (long long)NKV * HD, 0};
    g.v = {qkv + (NQ + NKV) * HD, qs, NKV, nullptr, nullptr, vc, (long long)NKV * HD, 0};
    g.n_tokens = T;
    g.head_dim = HD;
    g.cos_table = ct;
    g.sin_table = stb;
    g.positions = pos;
    g.rope_max_dim = HD / 2;
    g.table_rows = POS;
    g.eps = 1e-6f;
    bad |= L.qkv_rope_stage(&g);
    bad |= L.swiglu_q8(codes, scales, gate, up, T, HID, GS);
  };
  constexpr int kCalls = 4;
  hipEvent_t e0, e1;
  HIPCHECK(hipEventCreate(&e0));
  HIPCHECK(hipEventCreate(&e1));
  auto gpu_us = [&](auto run) {
    run();
    HIPCHECK(hipStreamSynchronize(st));
    HIPCHECK(hipEventRecord(e0, st));
    run();
    HIPCHECK(hipEventRecord(e1, st));
    HIPCHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    HIPCHECK(hipEventElapsedTime(&ms, e0, e1));
    return ms * 1e3 / N;
  };
  const double eager = gpu_us([&]() { for (int i = 0; i < N; ++i) step(); });
  HIPCHECK(hipStreamSynchronize(st));
  const auto h0 = std::chrono::steady_clock::now();
  for (int i = 0; i < N; ++i) step();
  const auto h1 = std::chrono::steady_clock::now();
  HIPCHECK(hipStreamSynchronize(st));
  const double host_call = std::chrono::duration<double, std::micro>(h1 - h0).count() / (N * kCalls);
  hipGraph_t g1, gn;
  hipGraphExec_t x1, xn;
  HIPCHECK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  step();
  HIPCHECK(hipStreamEndCapture(st, &g1));
  HIPCHECK(hipGraphInstantiate(&x1, g1, nullptr, nullptr, 0));
  HIPCHECK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  for (int i = 0; i < N; ++i) step();
  HIPCHECK(hipStreamEndCapture(st, &gn));
  HIPCHECK(hipGraphInstantiate(&xn, gn, nullptr, nullptr, 0));
  const double g_each = gpu_us([&]() { for (int i = 0; i < N; ++i) HIPCHECK(hipGraphLaunch(x1, st)); });
  const double g_all = gpu_us([&]() { HIPCHECK(hipGraphLaunch(xn, st)); });
  if (bad || L.get_last_error()) {
    printf("Fail: a call failed (%d)\n", bad);
    exit(1);
  }
  printf("Pass: decode step, tokens=%d (%d calls) iterations=%d\n", T, kCalls, N);
  printf("  eager %.2f us / step (host %.2f us / call), graph per step %.2f us, graph of %d steps %.2f us / step\n",
         eager, host_call, g_each, N, g_all);
  printf("{\"kernel\": \"decode_step\", \"tokens\": %d, \"eager_us\": %.3f, \"host_us_per_call\": %.3f, "
         "\"graph_per_step_us\": %.3f, \"graph_all_steps_us\": %.3f, \"steps\": %d}\n",
         T, eager, host_call, g_each, g_all, N);
  fflush(stdout);
  HIPCHECK(hipGraphExecDestroy(x1));
  HIPCHECK(hipGraphExecDestroy(xn));
  HIPCHECK(hipGraphDestroy(g1));
  HIPCHECK(hipGraphDestroy(gn));
  HIPCHECK(hipEventDestroy(e0));
  HIPCHECK(hipEventDestroy(e1));
  for (void *p : {(void *)tq, (void *)ts, (void *)out, (void *)normed, (void *)res, (void *)w, (void *)qkv, (void *)qw,
                  (void *)kw, (void *)gate, (void *)up, (void *)codes, (void *)scales, (void *)kc, (void *)vc,
                  (void *)ct, (void *)stb, (void *)ids, (void *)pos})
    HIPCHECK(hipFree(p));
}

int usage() {
  printf("usage: v7g_loadtest <libv7g.so> fused_add_rmsnorm|rmsnorm|add_inplace <rows> <dim> | rmsnorm_rope <tokens> <q_heads> "
         "<kv_heads> <head_dim> | swiglu <rows> <hidden> | swiglu_q8 <rows> <hidden> [gs] | embedding <tokens> "
         "<vocab> <dim> | rmsnorm_quantize|add_rmsnorm_quantize <rows> <dim> [gs] | kv_pack|kv_pack_kv <tokens> <kv_dim> "
         "| qkv_stage <tokens> <q_heads> <kv_heads> <head_dim> | rope_only <tokens> <q_heads> <kv_heads> <head_dim> "
         "[bias] | configs | next | models [tokens] [name] | decode [tokens]   [--iterations N] [--time secs] "
         "[--no-rotate] [--per-row]\n");
  return 1;
}

}  // namespace

int main(int argc, char **argv) {
  if (argc < 3) return usage();
  Opts opt;
  std::vector<std::string> pos;
  for (int i = 2; i < argc; ++i) {
    if (!strcmp(argv[i], "--iterations") && i + 1 < argc)
      opt.iterations = atoi(argv[++i]);
    else if (!strcmp(argv[i], "--time") && i + 1 < argc)
      opt.seconds = atof(argv[++i]);
    else if (!strcmp(argv[i], "--no-rotate"))
      opt.rotate = false;
    else if (!strcmp(argv[i], "--per-row"))
      opt.per_row = true;
    else
      pos.push_back(argv[i]);
  }
  if (pos.empty() || opt.iterations < 1) return usage();
  // The mode and its positional arguments are checked before the library or the GPU is touched.
  static const struct {
    const char *mode;
    size_t min_args;  // positional arguments including the mode
  } kModes[] = {{"fused_add_rmsnorm", 3}, {"rmsnorm", 3}, {"add_inplace", 3}, {"rmsnorm_rope", 5}, {"swiglu", 3}, {"swiglu_q8", 3}, {"embedding", 4},
                {"rmsnorm_quantize", 3}, {"add_rmsnorm_quantize", 3}, {"kv_pack", 3}, {"kv_pack_kv", 3},
                {"qkv_stage", 5}, {"rope_only", 5}, {"models", 1}, {"next", 1}, {"configs", 1}, {"decode", 1}};
  bool known = false;
  for (const auto &md : kModes) known = known || (pos[0] == md.mode && pos.size() >= md.min_args);
  if (!known) return usage();
  for (size_t i = 1; i < pos.size(); ++i) {
    const bool model_name = pos[0] == "models" && i == 2;
    if (!model_name && atoi(pos[i].c_str()) <= 0 && !(pos[0] == "rope_only" && i == 5)) return usage();
  }
  if (pos[0] == "models" && pos.size() >= 3) {
    bool found = false;
    for (const ModelShape &m : kModels) found = found || pos[2] == m.name;
    if (!found) {
      printf("Fail: no model shape named %s; the shapes:", pos[2].c_str());
      for (const ModelShape &m : kModels) printf(" %s", m.name);
      printf("\n");
      return 1;
    }
  }
  Lib L;
  if (load(argv[1], L)) return 1;
  if (L.init()) {
    printf("Fail: v7g_init\n");
    return 1;
  }
  hipStream_t st;
  HIPCHECK(hipStreamCreate(&st));
  L.set_stream(st);
  {
    int dev = 0;
    hipDeviceProp_t prop;
    HIPCHECK(hipGetDevice(&dev));
    HIPCHECK(hipGetDeviceProperties(&prop, dev));
    printf("device %d: %s (%s), %d CUs; host cores %u\n", dev, prop.name, prop.gcnArchName, prop.multiProcessorCount,
           std::thread::hardware_concurrency());
  }
  auto num = [&](size_t i, int dflt) { return i < pos.size() ? atoi(pos[i].c_str()) : dflt; };
  const std::string k = pos[0];
  if (k == "fused_add_rmsnorm" && pos.size() >= 3)
    run_add_rmsnorm(L, st, num(1, 0), num(2, 0), opt);
  else if (k == "rmsnorm" && pos.size() >= 3)
    run_rmsnorm(L, st, num(1, 0), num(2, 0), opt);
  else if (k == "add_inplace" && pos.size() >= 3)
    run_add_inplace(L, st, num(1, 0), num(2, 0), opt);
  else if (k == "rmsnorm_rope" && pos.size() >= 5)
    run_rope(L, st, num(1, 0), num(2, 0), num(3, 0), num(4, 0), opt);
  else if (k == "swiglu" && pos.size() >= 3)
    run_swiglu(L, st, num(1, 0), num(2, 0), 32, false, opt);
  else if (k == "swiglu_q8" && pos.size() >= 3)
    run_swiglu(L, st, num(1, 0), num(2, 0), num(3, 32), true, opt);
  else if (k == "embedding" && pos.size() >= 4)
    run_embedding(L, st, num(1, 0), num(2, 0), num(3, 0), opt);
  else if (k == "rmsnorm_quantize" && pos.size() >= 3)
    run_norm_q8(L, st, num(1, 0), num(2, 0), num(3, 64), false, opt);
  else if (k == "add_rmsnorm_quantize" && pos.size() >= 3)
    run_norm_q8(L, st, num(1, 0), num(2, 0), num(3, 64), true, opt);
  else if (k == "kv_pack" && pos.size() >= 3)
    run_kv_pack(L, st, num(1, 0), num(2, 0), false, opt);
  else if (k == "kv_pack_kv" && pos.size() >= 3)
    run_kv_pack(L, st, num(1, 0), num(2, 0), true, opt);
  else if (k == "qkv_stage" && pos.size() >= 5)
    run_qkv_stage(L, st, num(1, 0), num(2, 0), num(3, 0), num(4, 0), opt);
  else if (k == "rope_only" && pos.size() >= 5)
    run_rope_only(L, st, num(1, 0), num(2, 0), num(3, 0), num(4, 0), num(5, 0) != 0, opt);
  else if (k == "decode") {
    if (pos.size() >= 2)
      run_decode(L, st, num(1, 1), opt);
    else
      for (int T : {1, 8, 32, 64, 256}) run_decode(L, st, T, opt);
  } else if (k == "models" && num(1, 8192) > 0)
    run_models(L, st, num(1, 8192), pos.size() >= 3 ? pos[2].c_str() : nullptr, opt);
  else if (k == "next") {
    // The widened rows at the Qwen3-8B T=8192 shape (dim 4096, 32 Q / 8 KV heads of 128).
    run_norm_q8(L, st, 8192, 4096, 64, false, opt);
    run_norm_q8(L, st, 8192, 4096, 64, true, opt);
    run_kv_pack(L, st, 8192, 1024, false, opt);
    run_kv_pack(L, st, 8192, 1024, true, opt);
    run_qkv_stage(L, st, 8192, 32, 8, 128, opt);
    run_rmsnorm(L, st, 8192, 4096, opt);
    run_add_inplace(L, st, 8192, 4096, opt);
  } else if (k == "configs") {
    // The benchmark configurations: C1 .. C4, then the four kernels of the
    // Qwen3-8B T=8192 per-layer chain (C5a .. C5d).
    run_add_rmsnorm(L, st, 512, 2048, opt);
    run_rope(L, st, 2048, 16, 8, 128, opt);
    run_swiglu(L, st, 4096, 6144, 32, false, opt);
    run_swiglu(L, st, 4096, 8192, 32, true, opt);
    run_embedding(L, st, 8192, 151936, 4096, opt);
    run_add_rmsnorm(L, st, 8192, 4096, opt);
    run_rope(L, st, 8192, 32, 8, 128, opt);
    run_swiglu(L, st, 8192, 12288, 32, true, opt);
  } else {
    return usage();
  }
  HIPCHECK(hipStreamDestroy(st));
  return 0;
}
