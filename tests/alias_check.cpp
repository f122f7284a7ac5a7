// alias_check.cpp -- brute-force check of v7g::spans_overlap (csrc/v7g_alias.h), host only.
//
// Random pairs of spans (1..6 rows, strides 1..40 bytes, row lengths up to the
// stride, bases in a 400-byte window) are compared against a byte-by-byte
// intersection of the bytes they cover.  Prints the pair count and the number
// of disagreements; exits 1 on any disagreement.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>

#include "../v7multiplikator_amd/csrc/v7g_alias.h"

static bool brute(const v7g::Span &a, const v7g::Span &b) {
  static unsigned char mark[1 << 12];
  memset(mark, 0, sizeof mark);
  const uintptr_t origin = 0x100000;
  for (long long r = 0; r < a.rows; ++r)
    for (long long i = 0; i < a.row_bytes; ++i) mark[a.base - origin + r * a.stride + i] = 1;
  for (long long r = 0; r < b.rows; ++r)
    for (long long i = 0; i < b.row_bytes; ++i)
      if (mark[b.base - origin + r * b.stride + i]) return true;
  return false;
}

int main(int argc, char **argv) {
  const long long pairs = argc > 1 ? atoll(argv[1]) : 200000;
  std::mt19937_64 g(12345);
  auto pick = [&](long long lo, long long hi) { return lo + (long long)(g() % (unsigned long long)(hi - lo + 1)); };
  long long bad = 0, hits = 0;
  for (long long n = 0; n < pairs; ++n) {
    v7g::Span s[2];
    const bool same_stride = (n & 1) == 0;
    const long long common = pick(1, 40);
    for (auto &x : s) {
      x.rows = pick(1, 6);
      const long long stride = same_stride ? common : pick(1, 40);
      x.row_bytes = pick(1, stride);
      x.stride = x.rows > 1 ? stride : 0;
      x.base = 0x100000 + pick(0, 400);
    }
    const bool want = brute(s[0], s[1]);
    const bool got = v7g::spans_overlap(s[0], s[1]);
    hits += want;
    // Spans of different strides are compared by their extents: a reported
    // overlap may be a false alarm there, a missed one never.
    const bool exact = s[0].rows == 1 || s[1].rows == 1 || s[0].stride == s[1].stride;
    if (exact ? got != want : (want && !got)) {
      if (bad < 5)
        printf("disagree: a{%lu,%lld,%lld,%lld} b{%lu,%lld,%lld,%lld} want %d got %d\n", (unsigned long)s[0].base,
               s[0].rows, s[0].stride, s[0].row_bytes, (unsigned long)s[1].base, s[1].rows, s[1].stride,
               s[1].row_bytes, want, got);
      ++bad;
    }
    if (got != v7g::spans_overlap(s[1], s[0])) {
      if (bad < 5) printf("asymmetric result\n");
      ++bad;
    }
  }
  printf("pairs %lld overlapping %lld disagreements %lld\n", pairs, hits, bad);
  return bad ? 1 : 0;
}
