// fp_env.hip -- does gfx950 arithmetic in the library's flush mode equal x86
// SSE arithmetic under MXCSR FTZ+DAZ, the reference's mode?
//
//   v7g_fp_env [--count N]
//
// Built with the library's flags (f32 denormals flushed, -ffp-contract=off).
// N operand triples (default 2^20) concentrated at the denormal boundary:
// denormal operands, products and sums that land around 2^-126, quotients
// below it.  Each operation the kernels use runs on the GPU and, on the host,
// as the SSE instruction the reference uses with MXCSR |= 0x8040; one line per
// operation with its mismatch count (a NaN matches any NaN); the exit status
// is 1 if any operation differs.
#include <hip/hip_runtime.h>
#include <immintrin.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace {

#define CHECK(x)                                                                 \
  do {                                                                           \
    hipError_t e_ = (x);                                                         \
    if (e_ != hipSuccess) {                                                      \
      fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));             \
      exit(2);                                                                   \
    }                                                                            \
  } while (0)

float bf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
uint32_t fb(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

enum { MUL, ADD, SUB, FMA, DIV, RCP, SQRT, CMPGT, MAXMIN, MED3, F16, N_OPS };
const char *kNames[N_OPS] = {"mul (vmulss)", "add (vaddss)", "sub (vsubss)", "fma (vfmadd)", "div (vdivss)",
                             "1/x (vdivss)", "sqrt (vsqrtss)", "compare > (vcomiss)",
                             "max(x,-80) then min(.,80) (vmaxss, vminss)", "med3(x,-80,80) (vmaxss, vminss)",
                             "binary16 (vcvtps2ph imm 0)"};

__global__ void ops_kernel(const float *a, const float *b, const float *c, uint32_t *out, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float x = a[i], y = b[i], z = c[i];
  uint32_t *o = out + (size_t)i * N_OPS;
  o[MUL] = __builtin_bit_cast(uint32_t, x * y);
  o[ADD] = __builtin_bit_cast(uint32_t, x + y);
  o[SUB] = __builtin_bit_cast(uint32_t, x - y);
  o[FMA] = __builtin_bit_cast(uint32_t, __builtin_fmaf(x, y, z));
  o[DIV] = __builtin_bit_cast(uint32_t, x / y);
  o[RCP] = __builtin_bit_cast(uint32_t, 1.0f / y);
  o[SQRT] = __builtin_bit_cast(uint32_t, __builtin_sqrtf(__builtin_fabsf(x)));
  o[CMPGT] = x > y ? 1u : 0u;
  o[MAXMIN] = __builtin_bit_cast(uint32_t, __builtin_fminf(__builtin_fmaxf(x, -80.0f), 80.0f));
  o[MED3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_fmed3f(x, -80.0f, 80.0f));
  o[F16] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

__attribute__((target("fma,f16c,sse4.1"))) void host_ops(const float *a, const float *b, const float *c,
                                                         uint32_t *out, int n) {
  const unsigned old = _mm_getcsr();
  _mm_setcsr(old | 0x8040u);
  const __m128 absmask = _mm_castsi128_ps(_mm_set1_epi32(0x7fffffff));
  for (int i = 0; i < n; ++i) {
    const __m128 x = _mm_set_ss(a[i]), y = _mm_set_ss(b[i]), z = _mm_set_ss(c[i]);
    uint32_t *o = out + (size_t)i * N_OPS;
    o[MUL] = fb(_mm_cvtss_f32(_mm_mul_ss(x, y)));
    o[ADD] = fb(_mm_cvtss_f32(_mm_add_ss(x, y)));
    o[SUB] = fb(_mm_cvtss_f32(_mm_sub_ss(x, y)));
    o[FMA] = fb(_mm_cvtss_f32(_mm_fmadd_ss(x, y, z)));
    o[DIV] = fb(_mm_cvtss_f32(_mm_div_ss(x, y)));
    o[RCP] = fb(_mm_cvtss_f32(_mm_div_ss(_mm_set_ss(1.0f), y)));
    o[SQRT] = fb(_mm_cvtss_f32(_mm_sqrt_ss(_mm_and_ps(x, absmask))));
    o[CMPGT] = (uint32_t)_mm_comigt_ss(x, y) & 1u;
    const __m128 cl = _mm_min_ss(_mm_max_ss(x, _mm_set_ss(-80.0f)), _mm_set_ss(80.0f));
    o[MAXMIN] = fb(_mm_cvtss_f32(cl));
    o[MED3] = o[MAXMIN];
    o[F16] = (uint32_t)(uint16_t)_mm_extract_epi16(_mm_cvtps_ph(x, 0), 0);
  }
  _mm_setcsr(old);
}

bool is_nan(uint32_t u) { return (u & 0x7fffffffu) > 0x7f800000u; }

}  // namespace

int main(int argc, char **argv) {
  int n = 1 << 20;
  for (int i = 1; i < argc; ++i)
    if (!strcmp(argv[i], "--count") && i + 1 < argc) n = atoi(argv[++i]);
  if (n < 1 || n > (1 << 24)) {
    fprintf(stderr, "usage: v7g_fp_env [--count N], 1 <= N <= 2^24\n");
    return 2;
  }
  std::vector<float> a(n), b(n), c(n);
  uint64_t s = 0x9E3779B97F4A7C15ull;
  auto rnd = [&]() { s ^= s << 13; s ^= s >> 7; s ^= s << 17; return s; };
  auto mk = [&](int e) {  // random significand and sign, biased exponent e (0: denormal)
    return bf((uint32_t)(rnd() & 1) << 31 | (uint32_t)e << 23 | (uint32_t)(rnd() & 0x7fffff));
  };
  for (int i = 0; i < n; ++i) {
    switch ((int)(rnd() % 6)) {
      case 0: a[i] = mk(0); b[i] = mk(117 + (int)(rnd() % 20)); c[i] = mk(0); break;       // denormal x
      case 1: {                                                                           // x*y near 2^-126
        const int e1 = 31 + (int)(rnd() % 60);
        a[i] = mk(e1); b[i] = mk(127 - e1 + (int)(rnd() % 3)); c[i] = mk(1 + (int)(rnd() % 3));
        break;
      }
      case 2: a[i] = mk(1 + (int)(rnd() % 2)); b[i] = mk(1 + (int)(rnd() % 2)); c[i] = mk(1); break;  // tiny sums
      case 3: a[i] = mk(120 + (int)(rnd() % 20)); b[i] = mk(1 + (int)(rnd() % 250)); c[i] = mk(0); break;
      case 4: a[i] = mk(1 + (int)(rnd() % 8)); b[i] = mk(120 + (int)(rnd() % 15)); c[i] = mk(1); break;  // x/y tiny
      default: a[i] = mk(0); b[i] = mk(0); c[i] = mk(0); break;
    }
  }
  std::vector<uint32_t> g((size_t)n * N_OPS), h((size_t)n * N_OPS);
  float *da, *db, *dc;
  uint32_t *dout;
  CHECK(hipMalloc(&da, n * sizeof(float)));
  CHECK(hipMalloc(&db, n * sizeof(float)));
  CHECK(hipMalloc(&dc, n * sizeof(float)));
  CHECK(hipMalloc(&dout, (size_t)n * N_OPS * sizeof(uint32_t)));
  CHECK(hipMemcpy(da, a.data(), n * sizeof(float), hipMemcpyHostToDevice));
  CHECK(hipMemcpy(db, b.data(), n * sizeof(float), hipMemcpyHostToDevice));
  CHECK(hipMemcpy(dc, c.data(), n * sizeof(float), hipMemcpyHostToDevice));
  hipLaunchKernelGGL(ops_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, 0, da, db, dc, dout, n);
  CHECK(hipGetLastError());
  CHECK(hipMemcpy(g.data(), dout, (size_t)n * N_OPS * sizeof(uint32_t), hipMemcpyDeviceToHost));
  host_ops(a.data(), b.data(), c.data(), h.data(), n);
  long long total = 0;
  for (int op = 0; op < N_OPS; ++op) {
    long long bad = 0;
    int shown = 0;
    for (int i = 0; i < n; ++i) {
      const uint32_t gv = g[(size_t)i * N_OPS + op], hv = h[(size_t)i * N_OPS + op];
      const bool floaty = op != CMPGT && op != F16;
      if (gv == hv || (floaty && is_nan(gv) && is_nan(hv))) continue;
      ++bad;
      if (shown++ < 3)
        printf("  %s: x=%08x y=%08x z=%08x gpu=%08x x86=%08x\n", kNames[op], fb(a[i]), fb(b[i]), fb(c[i]), gv, hv);
    }
    printf("%-44s mismatches %lld of %d\n", kNames[op], bad, n);
    total += bad;
  }
  CHECK(hipFree(da));
  CHECK(hipFree(db));
  CHECK(hipFree(dc));
  CHECK(hipFree(dout));
  return total ? 1 : 0;
}
