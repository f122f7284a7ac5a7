// v7g_rope_tables.cpp -- host RoPE cos/sin tables for v7s_rope_init and the
// v7g_*rope_tables* / v7g_rope_init* entries (x86-64 host code, g++).
#include "v7g_rope_tables.h"

#include <algorithm>
#include <thread>
#include <vector>

// Host RoPE table builder: src/asm/fused_f32_kernel.inc:69-303.  The
// reference builds its tables with x87 instructions under control word 0x037F
// (64-bit significand, round to nearest, exceptions masked; :109-110,176-177);
// the builder issues the same instructions in the same order, so the tables
// carry the same bits.  The library's host is x86-64 (the MI355X platforms).
static_assert(sizeof(long double) >= 10, "the RoPE table builder needs the x87 80-bit format");

namespace {

long double x87_fyl2x(long double x, long double y) {  // y * log2(x)
  long double r;
  __asm__("fyl2x" : "=t"(r) : "0"(x), "u"(y) : "st(1)");
  return r;
}
long double x87_frndint(long double x) {
  long double r;
  __asm__("frndint" : "=t"(r) : "0"(x));
  return r;
}
long double x87_f2xm1(long double x) {  // 2^x - 1, |x| <= 1
  long double r;
  __asm__("f2xm1" : "=t"(r) : "0"(x));
  return r;
}
long double x87_fscale(long double x, long double e) {  // x * 2^trunc(e)
  long double r;
  __asm__("fscale" : "=t"(r) : "0"(x), "u"(e));
  return r;
}
void x87_fsincos(long double a, long double &c, long double &s) {
  __asm__("fsincos" : "=t"(c), "=u"(s) : "0"(a));
}

// Sets the reference's x87 control word for the scope (per thread: x87 state is per thread).
struct X87Mode {
  unsigned short old;
  X87Mode() {
    unsigned short cw = 0x037F;
    __asm__ volatile("fnstcw %0" : "=m"(old));
    __asm__ volatile("fldcw %0" : : "m"(cw));
  }
  ~X87Mode() { __asm__ volatile("fldcw %0" : : "m"(old)); }
};

}  // namespace

namespace v7g {

// RBIT_CALC_INV_FREQ (:117-134): t = j/half, y = -t * log2(base) (fyl2x),
// i = frndint(y), freq = (f2xm1(y - i) + 1) * 2^i (fscale); extended precision.
static long double inv_freq_x87(float base, int j, int half) {
  const long double t = (long double)j / (long double)half;
  const long double y = x87_fyl2x((long double)base, -t);
  const long double i = x87_frndint(y);
  return x87_fscale(x87_f2xm1(y - i) + 1.0L, i);
}

// Plain tables (rope type 0, :120-147): freq_j = base^(-j/half), stored as a double.
std::vector<double> plain_freqs(int half, float base) {
  X87Mode mode;
  std::vector<double> freq(half);
  for (int j = 0; j < half; ++j) freq[j] = (double)inv_freq_x87(base, j, half);
  return freq;
}

// Llama 3 frequency scaling (rope type 1, :149-256), the values rounded to
// double where the reference stores them: wavelen_j = 2 pi / inv_j; below the
// high-frequency wavelength inv_j is kept, above the low-frequency wavelength
// it is divided by factor, and in between it is interpolated with
// smooth = (orig/wavelen - low) / (high - low).
std::vector<double> llama3_freqs(int half, float base, float factor, float low_freq_factor, float high_freq_factor,
                                 int orig_max_pos) {
  typedef long double X;
  X87Mode mode;
  const double two_pi = 6.28318530717958647692;
  const double f = factor, lo = low_freq_factor, hi = high_freq_factor, old = orig_max_pos;
  const double low_wl = (double)((X)old / (X)lo);
  const double high_wl = (double)((X)old / (X)hi);
  std::vector<double> freq(half);
  for (int j = 0; j < half; ++j) {
    const X inv_x = inv_freq_x87(base, j, half);
    const double inv = (double)inv_x;
    const double wavelen = (double)((X)two_pi / inv_x);
    const double ifl = wavelen > low_wl ? (double)((X)inv / (X)f) : inv;
    const double smooth = (double)(((X)old / (X)wavelen - (X)lo) / ((X)hi - (X)lo));
    const double smoothed = (double)((1.0L - (X)smooth) * ((X)ifl / (X)f) + (X)smooth * (X)ifl);
    const bool medium = wavelen >= high_wl && wavelen <= low_wl;
    freq[j] = medium ? smoothed : ifl;
  }
  return freq;
}

// The .rbit_outer / .rbit_inner fill (:257-303): angle = freq_j * pos in
// extended precision (fld qword, fmul qword), fsincos, each result rounded
// to float (fstp dword).  Positions are split over host threads.
void fill_tables(std::vector<float> &c, std::vector<float> &s, int n_pos, const std::vector<double> &freq) {
  const int half = (int)freq.size();
  c.resize((size_t)n_pos * half);
  s.resize((size_t)n_pos * half);
  unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  std::vector<std::thread> th;
  for (unsigned w = 0; w < nt; ++w) {
    th.emplace_back([&, w]() {
      X87Mode mode;
      for (int p = (int)w; p < n_pos; p += (int)nt)
        for (int j = 0; j < half; ++j) {
          long double cv, sv;
          x87_fsincos((long double)freq[j] * (long double)(double)p, cv, sv);
          c[(size_t)p * half + j] = (float)cv;
          s[(size_t)p * half + j] = (float)sv;
        }
    });
  }
  for (auto &t : th) t.join();
}

}  // namespace v7g
