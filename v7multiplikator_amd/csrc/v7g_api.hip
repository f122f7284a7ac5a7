// v7g_api.hip -- the C ABI of libv7g.so: argument validation, stream, errors,
// RoPE tables, and the launches.  Declarations and contracts: include/v7g_lib.h.
//
// The reference dispatches these kernels through its CPU job pool
// (DISPATCH_EXECUTE, src/asm/dispatch_execute.inc:5-93) or runs them on the
// caller thread; here every call validates on the host and enqueues one HIP
// launch on the library stream.  No entry allocates except the RoPE table
// builders.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <cmath>
#include <mutex>
#include <thread>
#include <vector>

#include "v7g_alias.h"
#include "v7g_rope_tables.h"
#include "v7g_internal.h"
#include "../../include/v7g_lib.h"

namespace {

// The launch stream belongs to the calling host thread: threads that drive
// different streams do not see each other's choice.
thread_local hipStream_t g_stream = nullptr;
std::atomic<float> g_eps{1e-6f};
std::atomic<int> g_err{V7G_OK};

std::mutex g_rope_mu;
float *g_rope_cos = nullptr;
float *g_rope_sin = nullptr;
int g_rope_half = 0;
int g_rope_npos = 0;

// The model's RoPE configuration, standing in for the model DB keys the
// reference's table builder reads (__sys_rope_type, __sys_rope_base and, for
// type 1, __sys_rope_factor, __sys_rope_low_freq_factor,
// __sys_rope_high_freq_factor, __sys_rope_orig_max_pos;
// src/asm/fused_f32_kernel.inc:49-64,97-110,149-170).  v7s_rope_init builds
// from it when it is set and from its own arguments when it is not.
struct RopeConfig {
  bool set = false;
  int type = 0;  // 0 plain, 1 Llama 3 scaled
  float base = 0.0f, factor = 0.0f, low = 0.0f, high = 0.0f;
  int orig_max_pos = 0;
};
std::mutex g_rope_cfg_mu;
RopeConfig g_rope_cfg;

constexpr int kRopeMaxPositions = 131072;  // ROPE_INTERNAL_MAX_SEQ_LEN, src/asm/fused_f32_kernel.inc:9
constexpr int kMaxNormDim = 16384;         // LDS row staging limit of the add+RMSNorm kernel

int fail(int code) {
  int expected = V7G_OK;
  g_err.compare_exchange_strong(expected, code);
  return code;
}

// Called after the launches of every launching entry: also disarms the timing
// events, which cover that one call.
int check_launch() {
  v7g::launch_events() = v7g::LaunchEvents{};
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? V7G_OK : fail(V7G_ERR_HIP);
}

bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Pointer checks: off unless V7G_CHECK_POINTERS=1 or v7g_set_pointer_checks(1).
std::atomic<int> g_ptr_checks{-1};

bool pointer_checks() {
  int on = g_ptr_checks.load(std::memory_order_relaxed);
  if (on < 0) {
    const char *e = std::getenv("V7G_CHECK_POINTERS");
    on = (e && e[0] == '1') ? 1 : 0;
    int unset = -1;
    g_ptr_checks.compare_exchange_strong(unset, on);
    on = g_ptr_checks.load();
  }
  return on == 1;
}

// Device memory of the current device, managed memory or pinned host memory.
bool device_accessible(const void *p) {
  hipPointerAttribute_t a;
  if (hipPointerGetAttributes(&a, p) != hipSuccess) {
    (void)hipGetLastError();  // an unknown pointer is an answer here, not a pending error
    return false;
  }
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  switch (a.type) {
    case hipMemoryTypeDevice:
    case hipMemoryTypeArray:
      return a.device == dev;
    case hipMemoryTypeHost:
    case hipMemoryTypeManaged:
    case hipMemoryTypeUnified:
      return true;
    default:
      return false;
  }
}

// V7G_ERR_ADDRESS if pointer checks are on and a non-null pointer fails them.
int check_ptrs(std::initializer_list<const void *> ps) {
  if (!pointer_checks()) return V7G_OK;
  for (const void *p : ps)
    if (p && !device_accessible(p)) return V7G_ERR_ADDRESS;
  return V7G_OK;
}

// V7G_ERR_ALIAS if an output shares a byte with another output or with an
// input (v7g_alias.h).  Entries that accept an exact in-place form leave the
// coinciding pair out of the lists.
int check_alias(std::initializer_list<v7g::Span> outs, std::initializer_list<v7g::Span> ins) {
  for (auto o = outs.begin(); o != outs.end(); ++o) {
    for (auto p = o + 1; p != outs.end(); ++p)
      if (v7g::spans_overlap(*o, *p)) return V7G_ERR_ALIAS;
    for (const v7g::Span &i : ins)
      if (v7g::spans_overlap(*o, i)) return V7G_ERR_ALIAS;
  }
  return V7G_OK;
}

bool overlap(const v7g::Span &a, const v7g::Span &b) { return v7g::spans_overlap(a, b); }

int check_add_rmsnorm(const float *o, const float *residual, const float *add, const float *weight, int rows, int dim) {
  if (rows < 0 || dim <= 0 || dim % 8 != 0 || dim > kMaxNormDim) return V7G_ERR_SHAPE;
  if (rows == 0) return V7G_OK;  // nothing to touch: empty tensors may carry NULL pointers
  if (!o || !residual || !add || !weight) return V7G_ERR_NULL;
  if (!al16(o) || !al16(residual) || !al16(add) || !al16(weight)) return V7G_ERR_ALIGN;
  // o may be residual (the row ends as o, as in the reference) or add (read
  // before o is written, and only by the row's own workgroup); nothing else overlaps.
  const long long bytes = (long long)rows * dim * 4;
  const v7g::Span O = v7g::flat_span(o, bytes), R = v7g::flat_span(residual, bytes), A = v7g::flat_span(add, bytes),
                  W = v7g::flat_span(weight, (long long)dim * 4);
  if ((o != residual && overlap(O, R)) || (o != add && overlap(O, A)) || overlap(R, A) || overlap(O, W) ||
      overlap(R, W))
    return V7G_ERR_ALIAS;
  return V7G_OK;
}

int check_rope_common(int n_tokens, int head_dim, const float *cos_table, const float *sin_table, int rope_max_dim,
                      int table_rows) {
  if (n_tokens < 0 || head_dim < 64 || head_dim > 512 || head_dim % 32 != 0) return V7G_ERR_SHAPE;
  if (rope_max_dim < head_dim / 2 || rope_max_dim % 4 != 0 || table_rows < 0) return V7G_ERR_SHAPE;
  if (n_tokens == 0) return V7G_OK;
  if (!cos_table || !sin_table) return V7G_ERR_NULL;
  if (!al16(cos_table) || !al16(sin_table)) return V7G_ERR_ALIGN;
  return V7G_OK;
}

// 8 lanes per head: the grid of n_tokens * heads_per_token heads must stay below 2^32 threads.
// heads_per_token is the sum of the sides' head counts, taken in 64 bits by the callers.
int check_rope_heads(int n_tokens, long long heads_per_token) {
  return (heads_per_token >= (1LL << 28) || (long long)n_tokens * heads_per_token >= (1LL << 28)) ? V7G_ERR_SHAPE
                                                                                                  : V7G_OK;
}

int check_rope_side(const float *buf, long long token_stride, int n_heads, int head_dim, const float *w,
                    int n_tokens) {
  if (n_heads <= 0 || token_stride % 4 != 0) return V7G_ERR_SHAPE;
  if (n_tokens > 1 && token_stride < (long long)n_heads * head_dim) return V7G_ERR_SHAPE;
  if (n_tokens == 0) return V7G_OK;
  if (!buf || !w) return V7G_ERR_NULL;
  if (!al16(buf) || !al16(w)) return V7G_ERR_ALIGN;
  return V7G_OK;
}

// The head stage's arguments: a side's f32 heads are updated in place (an
// output when written back, else an input), its binary16 rows are outputs;
// norm weights, biases, tables and positions are inputs.  Sides inside one
// fused QKV row share the token stride and pass when their heads are apart.
int check_rope_alias(const v7g::RopeSide *sides, int n_sides, int n_tokens, int head_dim, const float *cos_table,
                     const float *sin_table, const int32_t *positions, int rope_max_dim, int table_rows) {
  v7g::Span outs[6], ins[12];
  int no = 0, ni = 0;
  for (int i = 0; i < n_sides; ++i) {
    const v7g::RopeSide &sd = sides[i];
    const long long hb = (long long)sd.n_heads * head_dim;
    const v7g::Span f = v7g::row_span(sd.buf, n_tokens, sd.token_stride * 4, hb * 4);
    if (!sd.cache || sd.keep_f32)
      outs[no++] = f;
    else
      ins[ni++] = f;
    if (sd.cache) outs[no++] = v7g::row_span(sd.cache, n_tokens, sd.cache_stride * 2, hb * 2);
    ins[ni++] = v7g::flat_span(sd.norm_weight, (long long)head_dim * 4);
    ins[ni++] = v7g::flat_span(sd.bias, hb * 4);
  }
  const long long table_bytes = (long long)table_rows * rope_max_dim * 4;
  ins[ni++] = v7g::flat_span(cos_table, table_bytes);
  ins[ni++] = v7g::flat_span(sin_table, table_bytes);
  ins[ni++] = v7g::flat_span(positions, (long long)n_tokens * 4);
  for (int a = 0; a < no; ++a) {
    for (int b = a + 1; b < no; ++b)
      if (overlap(outs[a], outs[b])) return V7G_ERR_ALIAS;
    for (int b = 0; b < ni; ++b)
      if (overlap(outs[a], ins[b])) return V7G_ERR_ALIAS;
  }
  return V7G_OK;
}

// The RoPE table builders (x87, host only) live in v7g_rope_tables.cpp.
using v7g::fill_tables;
using v7g::llama3_freqs;
using v7g::plain_freqs;

int check_table_shape(int n_pos, int head_dim) {
  return (n_pos <= 0 || n_pos > kRopeMaxPositions || head_dim < 2 || head_dim % 2 != 0 || head_dim > 1024)
             ? V7G_ERR_SHAPE
             : V7G_OK;
}

int check_tables_apart(const float *cos_table, const float *sin_table, int n_pos, int head_dim) {
  const long long bytes = (long long)n_pos * (head_dim / 2) * 4;
  return overlap(v7g::flat_span(cos_table, bytes), v7g::flat_span(sin_table, bytes)) ? V7G_ERR_ALIAS : V7G_OK;
}

// base^(-j/half) needs a positive finite base (the builder takes its log2).
int check_rope_base(float base) { return (base > 0.0f && std::isfinite(base)) ? V7G_OK : V7G_ERR_SHAPE; }

int check_llama3(float factor, float low_freq_factor, float high_freq_factor, int orig_max_pos) {
  const bool ok = factor > 0.0f && low_freq_factor > 0.0f && high_freq_factor > low_freq_factor &&
                  orig_max_pos > 0 && std::isfinite(factor) && std::isfinite(high_freq_factor);
  return ok ? V7G_OK : V7G_ERR_SHAPE;
}

int copy_tables(float *cos_table, float *sin_table, const std::vector<float> &c, const std::vector<float> &s) {
  const size_t bytes = c.size() * sizeof(float);
  if (hipMemcpy(cos_table, c.data(), bytes, hipMemcpyHostToDevice) != hipSuccess) return V7G_ERR_HIP;
  if (hipMemcpy(sin_table, s.data(), bytes, hipMemcpyHostToDevice) != hipSuccess) return V7G_ERR_HIP;
  return V7G_OK;
}

// Allocates library-owned tables from freq and publishes them, releasing the
// previous ones (v7s_rope_init owns its tables, fused_dispatch.inc:58-76).
int own_tables(int n_pos, const std::vector<double> &freq) {
  std::lock_guard<std::mutex> lk(g_rope_mu);
  if (g_rope_cos) {
    // Launches already queued, on any host thread's stream, may still read
    // the old tables: wait for the whole device before releasing them.
    if (hipDeviceSynchronize() != hipSuccess) return V7G_ERR_HIP;
    (void)hipFree(g_rope_cos);
    (void)hipFree(g_rope_sin);
    g_rope_cos = g_rope_sin = nullptr;
    g_rope_half = g_rope_npos = 0;
  }
  const int half = (int)freq.size();
  const size_t bytes = (size_t)n_pos * half * sizeof(float);
  float *c = nullptr, *s = nullptr;
  if (hipMalloc(&c, bytes) != hipSuccess) return V7G_ERR_HIP;
  if (hipMalloc(&s, bytes) != hipSuccess) {
    (void)hipFree(c);
    return V7G_ERR_HIP;
  }
  std::vector<float> hc, hs;
  fill_tables(hc, hs, n_pos, freq);
  const int rc = copy_tables(c, s, hc, hs);
  if (rc != V7G_OK) {
    (void)hipFree(c);
    (void)hipFree(s);
    return rc;
  }
  g_rope_cos = c;
  g_rope_sin = s;
  g_rope_half = half;
  g_rope_npos = n_pos;
  return V7G_OK;
}

hipStream_t stream() { return g_stream; }

// Table rows 0..pos for the one-token drop-in entries, without overflowing at INT_MAX.
int rows_through(int pos) { return pos < 2147483647 ? pos + 1 : pos; }

}  // namespace

namespace v7g {
LaunchEvents &launch_events() {
  static thread_local LaunchEvents ev;
  return ev;
}
}  // namespace v7g

extern "C" {

// ---------------------------------------------------------------- control

int v7g_init(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(V7G_ERR_HIP);
  if (hipFree(nullptr) != hipSuccess) return fail(V7G_ERR_HIP);
  return V7G_OK;
}

void v7g_set_pointer_checks(int on) { g_ptr_checks.store(on ? 1 : 0); }
int v7g_get_pointer_checks(void) { return pointer_checks() ? 1 : 0; }
int v7g_check_pointer(const void *p) { return (p && device_accessible(p)) ? V7G_OK : V7G_ERR_ADDRESS; }

void v7g_set_stream(void *s) { g_stream = reinterpret_cast<hipStream_t>(s); }
void *v7g_get_stream(void) { return reinterpret_cast<void *>(g_stream); }

int v7g_time_next_call(void *start_event, void *stop_event) {
  v7g::launch_events() = v7g::LaunchEvents{reinterpret_cast<hipEvent_t>(start_event),
                                           reinterpret_cast<hipEvent_t>(stop_event)};
  return V7G_OK;
}

int v7g_sync(void) { return hipStreamSynchronize(stream()) == hipSuccess ? V7G_OK : fail(V7G_ERR_HIP); }

void v7g_set_rms_eps(float eps) { g_eps.store(eps); }
float v7g_get_rms_eps(void) { return g_eps.load(); }

int v7g_get_last_error(void) { return g_err.load(); }
void v7g_clear_last_error(void) { g_err.store(V7G_OK); }

const char *v7g_error_string(int code) {
  switch (code) {
    case V7G_OK: return "ok";
    case V7G_ERR_NULL: return "a required pointer is NULL";
    case V7G_ERR_SHAPE: return "a size violates the kernel contract";
    case V7G_ERR_ALIGN: return "a pointer is not aligned as the kernel needs";
    case V7G_ERR_HIP: return "the HIP runtime reported an error";
    case V7G_ERR_NO_TABLES: return "RoPE tables requested before v7s_rope_init";
    case V7G_ERR_ADDRESS: return "a pointer is not memory the current device can access";
    case V7G_ERR_ALIAS: return "an output overlaps another argument";
    default: return "unknown error";
  }
}

int v7g_build_rope_tables(float *cos_table, float *sin_table, int n_pos, int head_dim, float rope_base) {
  if (!cos_table || !sin_table) return fail(V7G_ERR_NULL);
  if (int rc = check_table_shape(n_pos, head_dim)) return fail(rc);
  if (int rc = check_tables_apart(cos_table, sin_table, n_pos, head_dim)) return fail(rc);
  std::vector<float> c, s;
  fill_tables(c, s, n_pos, plain_freqs(head_dim / 2, rope_base));
  const int rc = copy_tables(cos_table, sin_table, c, s);
  return rc ? fail(rc) : V7G_OK;
}

int v7g_build_rope_tables_llama3(float *cos_table, float *sin_table, int n_pos, int head_dim, float rope_base,
                                 float factor, float low_freq_factor, float high_freq_factor, int orig_max_pos) {
  if (!cos_table || !sin_table) return fail(V7G_ERR_NULL);
  if (int rc = check_table_shape(n_pos, head_dim)) return fail(rc);
  if (int rc = check_llama3(factor, low_freq_factor, high_freq_factor, orig_max_pos)) return fail(rc);
  if (int rc = check_tables_apart(cos_table, sin_table, n_pos, head_dim)) return fail(rc);
  std::vector<float> c, s;
  fill_tables(c, s, n_pos,
              llama3_freqs(head_dim / 2, rope_base, factor, low_freq_factor, high_freq_factor, orig_max_pos));
  const int rc = copy_tables(cos_table, sin_table, c, s);
  return rc ? fail(rc) : V7G_OK;
}

int v7g_rope_init(int head_dim, float rope_base, int n_pos) {
  if (int rc = check_table_shape(n_pos, head_dim)) return fail(rc);
  const int rc = own_tables(n_pos, plain_freqs(head_dim / 2, rope_base));
  return rc ? fail(rc) : V7G_OK;
}

int v7g_rope_init_llama3(int head_dim, float rope_base, int n_pos, float factor, float low_freq_factor,
                         float high_freq_factor, int orig_max_pos) {
  if (int rc = check_table_shape(n_pos, head_dim)) return fail(rc);
  if (int rc = check_llama3(factor, low_freq_factor, high_freq_factor, orig_max_pos)) return fail(rc);
  const int rc = own_tables(
      n_pos, llama3_freqs(head_dim / 2, rope_base, factor, low_freq_factor, high_freq_factor, orig_max_pos));
  return rc ? fail(rc) : V7G_OK;
}

int v7g_set_rope_config(int rope_type, float rope_base, float factor, float low_freq_factor, float high_freq_factor,
                        int orig_max_pos) {
  if (rope_type != 0 && rope_type != 1) return fail(V7G_ERR_SHAPE);
  if (int rc = check_rope_base(rope_base)) return fail(rc);
  if (rope_type == 1)
    if (int rc = check_llama3(factor, low_freq_factor, high_freq_factor, orig_max_pos)) return fail(rc);
  RopeConfig c;
  c.set = true;
  c.type = rope_type;
  c.base = rope_base;
  if (rope_type == 1) {
    c.factor = factor;
    c.low = low_freq_factor;
    c.high = high_freq_factor;
    c.orig_max_pos = orig_max_pos;
  }
  std::lock_guard<std::mutex> lk(g_rope_cfg_mu);
  g_rope_cfg = c;
  return V7G_OK;
}

int v7g_get_rope_config(int *rope_type, float *rope_base, float *factor, float *low_freq_factor,
                        float *high_freq_factor, int *orig_max_pos) {
  RopeConfig c;
  {
    std::lock_guard<std::mutex> lk(g_rope_cfg_mu);
    c = g_rope_cfg;
  }
  if (!c.set) return 0;
  if (rope_type) *rope_type = c.type;
  if (rope_base) *rope_base = c.base;
  if (factor) *factor = c.factor;
  if (low_freq_factor) *low_freq_factor = c.low;
  if (high_freq_factor) *high_freq_factor = c.high;
  if (orig_max_pos) *orig_max_pos = c.orig_max_pos;
  return 1;
}

void v7g_clear_rope_config(void) {
  std::lock_guard<std::mutex> lk(g_rope_cfg_mu);
  g_rope_cfg = RopeConfig{};
}

int v7g_arith_selfcheck(unsigned long long *mismatches) {
  if (!mismatches) return fail(V7G_ERR_NULL);
  const int rc = v7g::arith_selfcheck(mismatches, stream());
  v7g::launch_events() = v7g::LaunchEvents{};
  return rc == 0 ? V7G_OK : fail(V7G_ERR_HIP);
}

int v7g_arith_selfcheck_noalloc(unsigned long long *mismatches, int checks) {
  if (!mismatches) return fail(V7G_ERR_NULL);
  if (checks <= 0 || checks > 0xF) return fail(V7G_ERR_SHAPE);  // four identities, four counters
  const int rc = v7g::arith_selfcheck_noalloc(mismatches, checks, stream());
  v7g::launch_events() = v7g::LaunchEvents{};
  return rc == 0 ? V7G_OK : fail(V7G_ERR_HIP);
}

int v7g_get_rope_tables(float **cos_table, float **sin_table, int *rope_max_dim, int *n_pos) {
  std::lock_guard<std::mutex> lk(g_rope_mu);
  if (!g_rope_cos) return fail(V7G_ERR_NO_TABLES);
  if (cos_table) *cos_table = g_rope_cos;
  if (sin_table) *sin_table = g_rope_sin;
  if (rope_max_dim) *rope_max_dim = g_rope_half;
  if (n_pos) *n_pos = g_rope_npos;
  return V7G_OK;
}

// ---------------------------------------------------------------- batched

int v7g_fused_add_rmsnorm(float *o, float *residual, const float *add, const float *weight, int rows, int dim,
                          float eps) {
  int rc = check_add_rmsnorm(o, residual, add, weight, rows, dim);
  if (rc) return fail(rc);
  if (rows == 0) return V7G_OK;
  if (int pc = check_ptrs({o, residual, add, weight})) return fail(pc);
  v7g::launch_fused_add_rmsnorm(o, residual, add, weight, rows, dim, eps, stream());
  return check_launch();
}

int v7g_rmsnorm(float *o, const float *x, const float *weight, int rows, int dim, float eps) {
  if (rows < 0 || dim <= 0 || dim % 32 != 0 || dim > kMaxNormDim) return fail(V7G_ERR_SHAPE);
  if (rows == 0) return V7G_OK;
  if (!o || !x || !weight) return fail(V7G_ERR_NULL);
  if (!al16(o) || !al16(x) || !al16(weight)) return fail(V7G_ERR_ALIGN);
  {
    const long long bytes = (long long)rows * dim * 4;
    const v7g::Span O = v7g::flat_span(o, bytes), X = v7g::flat_span(x, bytes),
                    W = v7g::flat_span(weight, (long long)dim * 4);
    if ((o != x && overlap(O, X)) || overlap(O, W)) return fail(V7G_ERR_ALIAS);  // o == x: in place
  }
  if (int pc = check_ptrs({o, x, weight})) return fail(pc);
  v7g::launch_rmsnorm(o, x, weight, rows, dim, eps, stream());
  return check_launch();
}

static int check_norm_q8(const int8_t *out_q, const float *out_s, const float *x, const float *weight, int rows,
                         int dim, int gs) {
  if (rows < 0 || dim <= 0 || dim > kMaxNormDim || (gs != 32 && gs != 64) || dim % gs != 0) return V7G_ERR_SHAPE;
  if (rows == 0) return V7G_OK;
  if (!out_q || !out_s || !x || !weight) return V7G_ERR_NULL;
  if (((uintptr_t)out_q & 3u) || ((uintptr_t)out_s & 3u) || !al16(x) || !al16(weight)) return V7G_ERR_ALIGN;
  return V7G_OK;
}

// Codes and scales beside x (and add, for the fused form), never over them.
static int check_norm_q8_alias(const int8_t *out_q, const float *out_s, const float *x, const float *add,
                               const float *weight, int rows, int dim, int gs) {
  const long long n = (long long)rows * dim;
  const v7g::Span Q = v7g::flat_span(out_q, n), S = v7g::flat_span(out_s, n / gs * 4), X = v7g::flat_span(x, n * 4),
                  A = v7g::flat_span(add, n * 4), W = v7g::flat_span(weight, (long long)dim * 4);
  if (add) return check_alias({Q, S, X}, {A, W});  // the residual x is updated in place: an output
  return check_alias({Q, S}, {X, W});
}

int v7g_rmsnorm_quantize(int8_t *out_q, float *out_s, const float *x, const float *weight, int rows, int dim, int gs,
                         float eps) {
  int rc = check_norm_q8(out_q, out_s, x, weight, rows, dim, gs);
  if (!rc && rows > 0) rc = check_norm_q8_alias(out_q, out_s, x, nullptr, weight, rows, dim, gs);
  if (rc) return fail(rc);
  if (rows == 0) return V7G_OK;
  if (int pc = check_ptrs({out_q, out_s, x, weight})) return fail(pc);
  v7g::launch_rmsnorm_quantize(out_q, out_s, const_cast<float *>(x), nullptr, weight, rows, dim, gs, eps, stream());
  return check_launch();
}

int v7g_add_rmsnorm_quantize(int8_t *out_q, float *out_s, float *residual, const float *add, const float *weight,
                             int rows, int dim, int gs, float eps) {
  int rc = check_norm_q8(out_q, out_s, residual, weight, rows, dim, gs);
  if (!rc && rows > 0 && !add) rc = V7G_ERR_NULL;
  if (!rc && rows > 0 && !al16(add)) rc = V7G_ERR_ALIGN;
  if (!rc && rows > 0) rc = check_norm_q8_alias(out_q, out_s, residual, add, weight, rows, dim, gs);
  if (rc) return fail(rc);
  if (rows == 0) return V7G_OK;
  if (int pc = check_ptrs({out_q, out_s, residual, add, weight})) return fail(pc);
  v7g::launch_rmsnorm_quantize(out_q, out_s, residual, add, weight, rows, dim, gs, eps, stream());
  return check_launch();
}

int v7g_add_inplace(float *x, const float *y, long long n) {
  if (n < 0 || n >= (1LL << 40)) return fail(V7G_ERR_SHAPE);  // one float4 per thread: below 2^31 blocks
  if (n == 0) return V7G_OK;
  if (!x || !y) return fail(V7G_ERR_NULL);
  if (!al16(x) || !al16(y)) return fail(V7G_ERR_ALIGN);
  if (x != y && overlap(v7g::flat_span(x, n * 4), v7g::flat_span(y, n * 4))) return fail(V7G_ERR_ALIAS);
  if (int pc = check_ptrs({x, y})) return fail(pc);
  v7g::launch_add_inplace(x, y, n, stream());
  return check_launch();
}

int v7g_rmsnorm_rope_heads(float *buf, int n_tokens, long long token_stride, int n_heads, int head_dim,
                           const float *norm_weight, const float *cos_table, const float *sin_table,
                           const int32_t *positions, int pos0, int rope_max_dim, int table_rows, float eps) {
  int rc = check_rope_common(n_tokens, head_dim, cos_table, sin_table, rope_max_dim, table_rows);
  if (!rc) rc = check_rope_side(buf, token_stride, n_heads, head_dim, norm_weight, n_tokens);
  if (!rc) rc = check_rope_heads(n_tokens, n_heads);
  if (!rc && positions && ((uintptr_t)positions & 3u)) rc = V7G_ERR_ALIGN;
  if (rc) return fail(rc);
  if (n_tokens == 0) return V7G_OK;
  v7g::RopeSide side{buf, token_stride, n_heads, norm_weight};
  if (int ac = check_rope_alias(&side, 1, n_tokens, head_dim, cos_table, sin_table, positions, rope_max_dim,
                                table_rows))
    return fail(ac);
  if (int pc = check_ptrs({buf, norm_weight, cos_table, sin_table, positions})) return fail(pc);
  v7g::launch_rmsnorm_rope(&side, 1, n_tokens, head_dim, cos_table, sin_table, positions, pos0, rope_max_dim,
                           table_rows, eps, stream());
  return check_launch();
}

int v7g_qk_rmsnorm_rope(float *q, long long q_token_stride, int n_q_heads, const float *q_norm_weight, float *k,
                        long long k_token_stride, int n_kv_heads, const float *k_norm_weight, int n_tokens,
                        int head_dim, const float *cos_table, const float *sin_table, const int32_t *positions,
                        int pos0, int rope_max_dim, int table_rows, float eps) {
  int rc = check_rope_common(n_tokens, head_dim, cos_table, sin_table, rope_max_dim, table_rows);
  if (!rc) rc = check_rope_side(q, q_token_stride, n_q_heads, head_dim, q_norm_weight, n_tokens);
  if (!rc) rc = check_rope_side(k, k_token_stride, n_kv_heads, head_dim, k_norm_weight, n_tokens);
  if (!rc) rc = check_rope_heads(n_tokens, (long long)n_q_heads + n_kv_heads);
  if (!rc && positions && ((uintptr_t)positions & 3u)) rc = V7G_ERR_ALIGN;
  if (rc) return fail(rc);
  if (n_tokens == 0) return V7G_OK;
  v7g::RopeSide sides[2] = {{q, q_token_stride, n_q_heads, q_norm_weight},
                            {k, k_token_stride, n_kv_heads, k_norm_weight}};
  if (int ac = check_rope_alias(sides, 2, n_tokens, head_dim, cos_table, sin_table, positions, rope_max_dim,
                                table_rows))
    return fail(ac);
  if (int pc = check_ptrs({q, q_norm_weight, k, k_norm_weight, cos_table, sin_table, positions})) return fail(pc);
  v7g::launch_rmsnorm_rope(sides, 2, n_tokens, head_dim, cos_table, sin_table, positions, pos0, rope_max_dim,
                           table_rows, eps, stream());
  return check_launch();
}

int v7g_qk_rmsnorm_rope_kv(float *q, long long q_token_stride, int n_q_heads, const float *q_norm_weight, float *k,
                           long long k_token_stride, int n_kv_heads, const float *k_norm_weight, int n_tokens,
                           int head_dim, const float *cos_table, const float *sin_table, const int32_t *positions,
                           int pos0, int rope_max_dim, int table_rows, float eps, uint16_t *k_cache,
                           long long k_cache_stride, int keep_k_f32) {
  v7g_qkv_stage st;
  memset(&st, 0, sizeof(st));
  st.q = {q, q_token_stride, n_q_heads, q_norm_weight, nullptr, nullptr, 0, 1};
  st.k = {k, k_token_stride, n_kv_heads, k_norm_weight, nullptr, k_cache, k_cache_stride, keep_k_f32};
  st.n_tokens = n_tokens;
  st.head_dim = head_dim;
  st.cos_table = cos_table;
  st.sin_table = sin_table;
  st.positions = positions;
  st.pos0 = pos0;
  st.rope_max_dim = rope_max_dim;
  st.table_rows = table_rows;
  st.eps = eps;
  if (n_tokens > 0 && !k_cache) return fail(V7G_ERR_NULL);
  return v7g_qkv_rope_stage(&st);
}

static int check_stage_side(const v7g_qkv_side &sd, int n_tokens, int head_dim, bool allow_norm, bool allow_cache) {
  if (sd.n_heads <= 0 || sd.token_stride % 4 != 0) return V7G_ERR_SHAPE;
  if (n_tokens > 1 && sd.token_stride < (long long)sd.n_heads * head_dim) return V7G_ERR_SHAPE;
  if ((sd.norm_weight && !allow_norm) || (sd.cache && !allow_cache)) return V7G_ERR_SHAPE;
  if (!sd.keep_f32 && !sd.cache) return V7G_ERR_SHAPE;  // nothing would be written
  if (sd.cache && (sd.cache_stride % 4 != 0 || (n_tokens > 1 && sd.cache_stride < (long long)sd.n_heads * head_dim)))
    return V7G_ERR_SHAPE;
  if (n_tokens == 0) return V7G_OK;
  if (!sd.buf) return V7G_ERR_NULL;
  if (!al16(sd.buf) || (sd.norm_weight && !al16(sd.norm_weight)) || (sd.bias && !al16(sd.bias)) ||
      ((uintptr_t)sd.cache & 7u))
    return V7G_ERR_ALIGN;
  return V7G_OK;
}

int v7g_qkv_rope_stage(const v7g_qkv_stage *st) {
  if (!st) return fail(V7G_ERR_NULL);
  const bool has_v = st->v.buf != nullptr;
  int rc = check_rope_common(st->n_tokens, st->head_dim, st->cos_table, st->sin_table, st->rope_max_dim,
                             st->table_rows);
  if (!rc) rc = check_stage_side(st->q, st->n_tokens, st->head_dim, true, false);
  if (!rc) rc = check_stage_side(st->k, st->n_tokens, st->head_dim, true, true);
  if (!rc && has_v) rc = check_stage_side(st->v, st->n_tokens, st->head_dim, false, true);
  if (!rc)
    rc = check_rope_heads(st->n_tokens, (long long)st->q.n_heads + st->k.n_heads + (has_v ? st->v.n_heads : 0));
  if (!rc && st->positions && ((uintptr_t)st->positions & 3u)) rc = V7G_ERR_ALIGN;
  if (rc) return fail(rc);
  if (st->n_tokens == 0) return V7G_OK;
  v7g::RopeSide sides[3];
  const v7g_qkv_side *src[3] = {&st->q, &st->k, &st->v};
  for (int i = 0; i < 3; ++i) {
    sides[i].buf = src[i]->buf;
    sides[i].token_stride = src[i]->token_stride;
    sides[i].n_heads = src[i]->n_heads;
    sides[i].norm_weight = src[i]->norm_weight;
    sides[i].bias = src[i]->bias;
    sides[i].cache = src[i]->cache;
    sides[i].cache_stride = src[i]->cache_stride;
    sides[i].keep_f32 = src[i]->keep_f32 != 0;
    sides[i].rotate = i < 2;
  }
  if (int ac = check_rope_alias(sides, has_v ? 3 : 2, st->n_tokens, st->head_dim, st->cos_table, st->sin_table,
                                st->positions, st->rope_max_dim, st->table_rows))
    return fail(ac);
  if (int pc = check_ptrs({st->q.buf, st->q.norm_weight, st->q.bias, st->k.buf, st->k.norm_weight, st->k.bias,
                           st->k.cache, st->cos_table, st->sin_table, st->positions}))
    return fail(pc);
  if (has_v)
    if (int pc = check_ptrs({st->v.buf, st->v.bias, st->v.cache})) return fail(pc);
  v7g::launch_rmsnorm_rope(sides, has_v ? 3 : 2, st->n_tokens, st->head_dim, st->cos_table, st->sin_table,
                           st->positions, st->pos0, st->rope_max_dim, st->table_rows, st->eps, stream());
  return check_launch();
}

int v7g_rope_only_heads(float *buf, int n_tokens, long long token_stride, int n_heads, int head_dim,
                        const float *cos_table, const float *sin_table, const int32_t *positions, int pos0,
                        int rope_max_dim, int table_rows) {
  int rc = check_rope_common(n_tokens, head_dim, cos_table, sin_table, rope_max_dim, table_rows);
  if (!rc) {
    if (n_heads <= 0 || token_stride % 4 != 0 || (n_tokens > 1 && token_stride < (long long)n_heads * head_dim))
      rc = V7G_ERR_SHAPE;
    else if (n_tokens > 0 && !buf)
      rc = V7G_ERR_NULL;
    else if (n_tokens > 0 && !al16(buf))
      rc = V7G_ERR_ALIGN;
  }
  if (!rc) rc = check_rope_heads(n_tokens, n_heads);
  if (!rc && positions && ((uintptr_t)positions & 3u)) rc = V7G_ERR_ALIGN;
  if (rc) return fail(rc);
  if (n_tokens == 0) return V7G_OK;
  v7g::RopeSide side{buf, token_stride, n_heads, nullptr};
  if (int ac = check_rope_alias(&side, 1, n_tokens, head_dim, cos_table, sin_table, positions, rope_max_dim,
                                table_rows))
    return fail(ac);
  if (int pc = check_ptrs({buf, cos_table, sin_table, positions})) return fail(pc);
  v7g::launch_rmsnorm_rope(&side, 1, n_tokens, head_dim, cos_table, sin_table, positions, pos0, rope_max_dim,
                           table_rows, 0.0f, stream());
  return check_launch();
}

int v7g_kv_pack_f16(uint16_t *dst, long long dst_stride, const float *src, long long src_stride, int rows,
                    int row_len) {
  if (rows < 0 || row_len <= 0 || row_len % 4 != 0 || dst_stride % 4 != 0 || src_stride % 4 != 0)
    return fail(V7G_ERR_SHAPE);
  if (rows > 1 && (dst_stride < row_len || src_stride < row_len)) return fail(V7G_ERR_SHAPE);
  if ((long long)rows * (row_len / 4) >= (1LL << 32) - 256) return fail(V7G_ERR_SHAPE);
  if (rows == 0) return V7G_OK;
  if (!dst || !src) return fail(V7G_ERR_NULL);
  if (((uintptr_t)dst & 7u) || !al16(src)) return fail(V7G_ERR_ALIGN);
  if (overlap(v7g::row_span(dst, rows, dst_stride * 2, (long long)row_len * 2),
              v7g::row_span(src, rows, src_stride * 4, (long long)row_len * 4)))
    return fail(V7G_ERR_ALIAS);
  if (int pc = check_ptrs({dst, src})) return fail(pc);
  v7g::launch_kv_pack_f16(dst, dst_stride, src, src_stride, rows, row_len, stream());
  return check_launch();
}

int v7g_kv_pack_f16_kv(uint16_t *k_dst, long long k_dst_stride, uint16_t *v_dst, long long v_dst_stride,
                       const float *k_src, const float *v_src, long long src_stride, int rows, int row_len) {
  if (rows < 0 || row_len <= 0 || row_len % 4 != 0 || k_dst_stride % 4 != 0 || v_dst_stride % 4 != 0 ||
      src_stride % 4 != 0)
    return fail(V7G_ERR_SHAPE);
  if (rows > 1 && (k_dst_stride < row_len || v_dst_stride < row_len || src_stride < row_len))
    return fail(V7G_ERR_SHAPE);
  if ((long long)rows * (row_len / 4) >= (1LL << 32) - 256) return fail(V7G_ERR_SHAPE);
  if (rows == 0) return V7G_OK;
  if (!k_dst || !v_dst || !k_src || !v_src) return fail(V7G_ERR_NULL);
  if (((uintptr_t)k_dst & 7u) || ((uintptr_t)v_dst & 7u) || !al16(k_src) || !al16(v_src)) return fail(V7G_ERR_ALIGN);
  {
    const long long rb = (long long)row_len;
    const v7g::Span K = v7g::row_span(k_dst, rows, k_dst_stride * 2, rb * 2),
                    V = v7g::row_span(v_dst, rows, v_dst_stride * 2, rb * 2);
    if (check_alias({K, V}, {v7g::row_span(k_src, rows, src_stride * 4, rb * 4),
                             v7g::row_span(v_src, rows, src_stride * 4, rb * 4)}))
      return fail(V7G_ERR_ALIAS);
  }
  if (int pc = check_ptrs({k_dst, v_dst, k_src, v_src})) return fail(pc);
  v7g::launch_kv_pack2_f16(k_dst, k_dst_stride, v_dst, v_dst_stride, k_src, v_src, src_stride, rows, row_len,
                           stream());
  return check_launch();
}

int v7g_swiglu_f32(float *out, const float *gate, const float *up, long long n) {
  if (n < 0 || n >= (1LL << 40)) return fail(V7G_ERR_SHAPE);  // one float4 per thread: below 2^31 blocks
  if (n == 0) return V7G_OK;
  if (!out || !gate || !up) return fail(V7G_ERR_NULL);
  if (!al16(out) || !al16(gate) || !al16(up)) return fail(V7G_ERR_ALIGN);
  {
    // out == gate (the reference's in-place form) or out == up: each element is read before it is replaced
    const v7g::Span O = v7g::flat_span(out, n * 4);
    if ((out != gate && overlap(O, v7g::flat_span(gate, n * 4))) || (out != up && overlap(O, v7g::flat_span(up, n * 4))))
      return fail(V7G_ERR_ALIAS);
  }
  if (int pc = check_ptrs({out, gate, up})) return fail(pc);
  v7g::launch_swiglu_f32(out, gate, up, n, stream());
  return check_launch();
}

static int check_quant(const int8_t *out_q, const float *out_s, int rows, int row_len, int gs) {
  if (rows < 0 || row_len <= 0 || gs < 1 || gs > 4096) return V7G_ERR_SHAPE;
  if ((long long)rows * row_len >= (1LL << 40)) return V7G_ERR_SHAPE;
  // the general path runs one thread per group in 256-thread blocks: at most 2^30 blocks
  if ((long long)rows * ((row_len + gs - 1) / gs) >= (1LL << 38)) return V7G_ERR_SHAPE;
  if (rows == 0) return V7G_OK;
  if (!out_q || !out_s) return V7G_ERR_NULL;
  if ((uintptr_t)out_s & 3u) return V7G_ERR_ALIGN;
  return V7G_OK;
}

// Codes and scales in their own buffers: never over the inputs (the reference
// writes the SwiGLU row's codes into the retired up row, src/asm/prefill_q8.inc:1169-1180,
// after the SwiGLU pass has finished; the fused kernel reads up while it writes codes).
static int check_quant_alias(const int8_t *out_q, const float *out_s, const float *a, const float *b, int rows,
                             int row_len, int gs) {
  const long long n = (long long)rows * row_len, groups = (long long)rows * ((row_len + gs - 1) / gs);
  return check_alias({v7g::flat_span(out_q, n), v7g::flat_span(out_s, groups * 4)},
                     {v7g::flat_span(a, n * 4), v7g::flat_span(b, n * 4)});
}

int v7g_swiglu_q8(int8_t *out_q, float *out_s, const float *gate, const float *up, int rows, int hidden, int gs) {
  int rc = check_quant(out_q, out_s, rows, hidden, gs);
  if (!rc && rows > 0 && (!gate || !up)) rc = V7G_ERR_NULL;
  if (!rc && rows > 0) rc = check_quant_alias(out_q, out_s, gate, up, rows, hidden, gs);
  if (rc) return fail(rc);
  if (rows == 0) return V7G_OK;
  if (int pc = check_ptrs({out_q, out_s, gate, up})) return fail(pc);
  v7g::launch_quantize_q8(out_q, out_s, nullptr, gate, up, rows, hidden, gs, stream());
  return check_launch();
}

int v7g_quantize_q8(int8_t *out_q, float *out_s, const float *x, int rows, int row_len, int gs) {
  int rc = check_quant(out_q, out_s, rows, row_len, gs);
  if (!rc && rows > 0 && !x) rc = V7G_ERR_NULL;
  if (!rc && rows > 0) rc = check_quant_alias(out_q, out_s, x, nullptr, rows, row_len, gs);
  if (rc) return fail(rc);
  if (rows == 0) return V7G_OK;
  if (int pc = check_ptrs({out_q, out_s, x})) return fail(pc);
  v7g::launch_quantize_q8(out_q, out_s, x, nullptr, nullptr, rows, row_len, gs, stream());
  return check_launch();
}

int v7g_embedding_gather_q8(float *out, const int32_t *ids, int n_tokens, const int8_t *table_q,
                            const float *table_s, int dim, int vocab) {
  if (n_tokens < 0 || dim <= 0 || dim % 64 != 0 || vocab <= 0) return fail(V7G_ERR_SHAPE);
  if (n_tokens == 0) return V7G_OK;
  if (!out || !ids || !table_q || !table_s) return fail(V7G_ERR_NULL);
  // the one-workgroup-per-row form (rows below 256 codes, launches of 2^32 dwords or more) takes up to
  // ceil(dim/4096) workgroups per row: its grid stays below 2^24 workgroups
  if ((long long)n_tokens * ((dim / 4 + 1023) / 1024) >= (1LL << 24)) return fail(V7G_ERR_SHAPE);
  if (!al16(out) || ((uintptr_t)table_q & 3u) || ((uintptr_t)table_s & 3u) || ((uintptr_t)ids & 3u))
    return fail(V7G_ERR_ALIGN);
  {
    const long long cells = (long long)vocab * dim;
    if (check_alias({v7g::flat_span(out, (long long)n_tokens * dim * 4)},
                    {v7g::flat_span(ids, (long long)n_tokens * 4), v7g::flat_span(table_q, cells),
                     v7g::flat_span(table_s, cells / 64 * 4)}))
      return fail(V7G_ERR_ALIAS);
  }
  if (int pc = check_ptrs({out, ids, table_q, table_s})) return fail(pc);
  v7g::launch_embedding_gather(out, ids, n_tokens, table_q, table_s, dim, vocab, stream());
  return check_launch();
}

// ---------------------------------------------------------------- drop-in (ms_abi)

V7_ABI void v7s_fused_add_rmsnorm(float *o, float *residual, float *add, float *weight, int dim) {
  v7g_fused_add_rmsnorm(o, residual, add, weight, 1, dim, g_eps.load());
}

V7_ABI void v7s_rope_only_heads(float *buf, int n_heads, int head_dim, float *cos_table, float *sin_table, int pos,
                                int rope_max_dim) {
  if (pos < 0) {
    fail(V7G_ERR_SHAPE);
    return;
  }
  v7g_rope_only_heads(buf, 1, (long long)n_heads * head_dim, n_heads, head_dim, cos_table, sin_table, nullptr, pos,
                      rope_max_dim, rows_through(pos));
}

V7_ABI void v7s_kv_pack_f16(uint16_t *dest, float *src, int count) {
  // The reference's contract: count is a positive multiple of 8 (src/asm/kv_f16c.inc:6).
  if (count <= 0 || count % 8 != 0) {
    fail(V7G_ERR_SHAPE);
    return;
  }
  v7g_kv_pack_f16(dest, count, src, count, 1, count);
}

V7_ABI void v7s_rmsnorm(float *o, float *x, float *weight, int size) {
  v7g_rmsnorm(o, x, weight, 1, size, g_eps.load());
}

V7_ABI void v7s_rmsnorm_quantize(char *out_q, float *in_x, float *out_s, int n, float *weight) {
  v7g_rmsnorm_quantize(reinterpret_cast<int8_t *>(out_q), out_s, in_x, weight, 1, n, 64, g_eps.load());
}

V7_ABI void v7s_add_inplace(float *x, float *y, int n) {
  if (n < 0) {
    fail(V7G_ERR_SHAPE);
    return;
  }
  v7g_add_inplace(x, y, n);
}

V7_ABI void v7s_rmsnorm_rope_heads(float *buf, int n_heads, int head_dim, float *norm_weight, float *cos_table,
                                   float *sin_table, int pos, int rope_max_dim) {
  if (pos < 0) {
    fail(V7G_ERR_SHAPE);
    return;
  }
  // The caller's tables hold at least pos+1 rows (the reference offsets them by
  // pos*rope_max_dim without a bound).
  v7g_rmsnorm_rope_heads(buf, 1, (long long)n_heads * head_dim, n_heads, head_dim, norm_weight, cos_table, sin_table,
                         nullptr, pos, rope_max_dim, rows_through(pos), g_eps.load());
}

V7_ABI void v7s_qk_fork_heads(const v7g_qk_fork_args *desc) {
  if (!desc) {
    fail(V7G_ERR_NULL);
    return;
  }
  const v7g_qk_fork_args d = *desc;  // a host descriptor, as the reference's lives on its caller's stack
  if (d.pos < 0 || d.head_dim < 64 || d.head_dim % 32 != 0) {
    fail(V7G_ERR_SHAPE);
    return;
  }
  // cos/sin already point at row pos.  Hand the kernel a table of rows of head_dim/2 floats whose row
  // pos starts there: base = cos - pos*half, which lies inside the caller's table (its rows hold
  // rope_max_dim >= half floats), and the kernel reads only row pos.
  const int half = d.head_dim / 2;
  const uintptr_t back = (uintptr_t)d.pos * (uintptr_t)half * sizeof(float);
  const float *cos_base = d.cos ? reinterpret_cast<const float *>(reinterpret_cast<uintptr_t>(d.cos) - back) : nullptr;
  const float *sin_base = d.sin ? reinterpret_cast<const float *>(reinterpret_cast<uintptr_t>(d.sin) - back) : nullptr;
  v7g_rmsnorm_rope_heads(d.buf, 1, (long long)d.heads * d.head_dim, d.heads, d.head_dim, d.weight, cos_base,
                         sin_base, nullptr, d.pos, half, rows_through(d.pos), g_eps.load());
}

V7_ABI void v7d_quantize(char *out_q, float *in_x, float *out_s, int n) {
  if (n <= 0) {
    if (n < 0) fail(V7G_ERR_SHAPE);
    return;
  }
  v7g_quantize_q8(reinterpret_cast<int8_t *>(out_q), out_s, in_x, 1, n, 64);
}

V7_ABI void v7s_embedding_row(float *out, int token, int dim, v7g_q8_tensor *q_desc) {
  if (!q_desc || !out) {
    fail(V7G_ERR_NULL);
    return;
  }
  if (token < 0 || dim <= 0 || dim % 64 != 0) {
    fail(V7G_ERR_SHAPE);
    return;
  }
  // One row: offset the table to the token's row and gather id 0 of a
  // one-row table, so the kernel needs no device-side id.
  size_t base = (size_t)token * (size_t)dim;
  const int8_t *q = reinterpret_cast<const int8_t *>(q_desc->q) + base;
  const float *s = q_desc->s + (base >> 6);
  if (!al16(out) || ((uintptr_t)q & 3u) || ((uintptr_t)s & 3u)) {
    fail(V7G_ERR_ALIGN);
    return;
  }
  if (check_alias({v7g::flat_span(out, (long long)dim * 4)},
                  {v7g::flat_span(q, dim), v7g::flat_span(s, (long long)dim / 64 * 4)})) {
    fail(V7G_ERR_ALIAS);
    return;
  }
  if (int pc = check_ptrs({out, q, s})) {
    fail(pc);
    return;
  }
  v7g::launch_embedding_gather(out, nullptr, 1, q, s, dim, 1, stream());
  check_launch();
}

V7_ABI void v7s_swiglu_row(float *gate_inout, float *up, int hidden) {
  if (hidden < 0) {
    fail(V7G_ERR_SHAPE);
    return;
  }
  v7g_swiglu_f32(gate_inout, gate_inout, up, hidden);
}

V7_ABI void v7s_swiglu_quantize_row(char *out_q, float *gate, float *up, float *out_s, int hidden) {
  v7g_swiglu_q8(reinterpret_cast<int8_t *>(out_q), out_s, gate, up, 1, hidden, 64);
}

// The reference keeps only head_dim from its arguments and reads the base and
// the rope type from the model DB (src/asm/fused_dispatch.inc:58-76,
// fused_f32_kernel.inc:97-110): with a configuration set by
// v7g_set_rope_config the float argument is ignored likewise; without one the
// tables are plain, from rope_base.
V7_ABI void v7s_rope_init(int head_dim, float rope_base) {
  RopeConfig c;
  {
    std::lock_guard<std::mutex> lk(g_rope_cfg_mu);
    c = g_rope_cfg;
  }
  if (!c.set)
    v7g_rope_init(head_dim, rope_base, kRopeMaxPositions);
  else if (c.type == 1)
    v7g_rope_init_llama3(head_dim, c.base, kRopeMaxPositions, c.factor, c.low, c.high, c.orig_max_pos);
  else
    v7g_rope_init(head_dim, c.base, kRopeMaxPositions);
}

}  // extern "C"
