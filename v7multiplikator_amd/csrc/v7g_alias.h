// v7g_alias.h -- host-side overlap test of the memory two kernel arguments cover.
//
// Every kernel of the library reads its inputs and writes its outputs in one
// pass, with many workgroups in flight at once: an output that shares bytes
// with another argument is read and written by different workgroups in no
// fixed order, and the result depends on the schedule.  The entries in
// v7g_api.hip reject such calls before any launch (V7G_ERR_ALIAS), except the
// exact in-place forms each entry documents (an output equal to the input it
// replaces element by element).
//
// An argument covers `rows` rows of `row_bytes` bytes, row r starting at
// base + r * stride bytes (one row: a plain byte range).  Two arguments with
// the same row stride -- Q, K and V heads inside one fused QKV row, K and V
// cache rows -- are tested row against row, so interleaved but disjoint
// layouts pass; rows of different strides are tested by their whole extents.
#pragma once
#include <stdint.h>

namespace v7g {

struct Span {
  uintptr_t base;      // 0: the argument is absent (covers nothing)
  long long rows;      // >= 1 to cover anything
  long long stride;    // bytes from one row to the next (rows > 1: >= row_bytes, validated by the entries)
  long long row_bytes;
};

inline Span flat_span(const void *p, long long bytes) { return Span{(uintptr_t)p, 1, 0, bytes}; }

inline Span row_span(const void *p, long long rows, long long stride_bytes, long long row_bytes) {
  return Span{(uintptr_t)p, rows, rows > 1 ? stride_bytes : 0, row_bytes};
}

namespace alias_detail {
typedef __int128 I;
// floor(n / d) for d > 0.
inline I floor_div(I n, I d) {
  I q = n / d;
  if (n % d != 0 && n < 0) q -= 1;
  return q;
}
}  // namespace alias_detail

// True if some byte lies in both a and b.
inline bool spans_overlap(const Span &a, const Span &b) {
  using alias_detail::I;
  if (!a.base || !b.base || a.rows <= 0 || b.rows <= 0 || a.row_bytes <= 0 || b.row_bytes <= 0) return false;
  const I a_end = (I)a.base + (I)(a.rows - 1) * a.stride + a.row_bytes;
  const I b_end = (I)b.base + (I)(b.rows - 1) * b.stride + b.row_bytes;
  if (a_end <= (I)b.base || b_end <= (I)a.base) return false;  // the extents are apart
  if (a.rows == 1 && b.rows == 1) return true;
  if (a.rows > 1 && b.rows > 1 && a.stride != b.stride) return true;  // different strides: the extents decide
  // A common stride S > 0 (a one-row span takes the other's).  Row t of a and
  // row u of b share a byte iff -b.row_bytes < k*S + d < a.row_bytes with
  // k = u - t in [-(a.rows-1), b.rows-1] and d = b.base - a.base.  The left
  // bound rises with k: take the smallest k that meets it and test the right one.
  const I S = a.rows > 1 ? a.stride : b.stride;
  if (S <= 0) return true;
  const I d = (I)b.base - (I)a.base;
  I k = alias_detail::floor_div(-(I)b.row_bytes - d, S) + 1;
  if (k < -(I)(a.rows - 1)) k = -(I)(a.rows - 1);
  if (k > (I)(b.rows - 1)) return false;
  return k * S + d < (I)a.row_bytes;
}

}  // namespace v7g
