// Element offsets in split-head storage (llattn_heads_layout of include/llattn.h, HeadsMap of llattn_abi.h):
// element (r, c), r = b T + t, of a [rows][ld] token-row matrix sits at
//   heads_row(r) + heads_col(c) = (b n T + t) dh + (c / dh) T dh + c % dh     for c < n dh,
//   tail + r w + c'                                                          otherwise, tdh = 0,
//   tail + (b (w / tdh) T + t) tdh + (c' / tdh) T tdh + c' % tdh             otherwise, tdh > 0,
// with w = tail_ld = ld - n dh and c' = c - n dh.
// All offsets stay below 2^30 elements (checked by heads_map), so 32-bit arithmetic is exact.
#pragma once

#include "llattn_abi.h"

namespace llattn {

// x / d for x < 2^31 with d's reciprocal (m, s) from magic_div
__device__ __forceinline__ uint32_t fdiv(uint32_t x, uint32_t m, uint32_t s) { return (__umulhi(x, m) + x) >> s; }

// row term of a head column: (b n T + t) dh
__device__ __forceinline__ uint32_t heads_row(const HeadsMap& h, uint32_t r) {
  const uint32_t b = fdiv(r, h.mt, h.st);
  return (b * (uint32_t)(h.n - 1) * (uint32_t)h.T + r) * (uint32_t)h.dh;  // b n T + t = b (n - 1) T + r
}
// column term of a head column (c < cols): (c / dh) T dh + c % dh
__device__ __forceinline__ uint32_t heads_col(const HeadsMap& h, uint32_t c) {
  const uint32_t g = fdiv(c, h.md, h.sd);
  return g * (uint32_t)(h.T - 1) * (uint32_t)h.dh + c;  // g T dh + c - g dh
}
// element offset of (r, c) in either part
__device__ __forceinline__ uint32_t heads_off(const HeadsMap& h, uint32_t r, uint32_t c) {
  if ((int)c < h.cols) return heads_row(h, r) + heads_col(h, c);
  const uint32_t c2 = c - (uint32_t)h.cols;
  if (h.tdh == 0) return h.tail + r * (uint32_t)h.tail_ld + c2;
  // ((b w / tdh + g) T + t) tdh + c2 % tdh = b (w - tdh) T + r tdh + g (T - 1) tdh + c2 with g = c2 / tdh
  const uint32_t b = fdiv(r, h.mt, h.st), g = fdiv(c2, h.mtd, h.std);
  return h.tail + (b * (uint32_t)(h.tail_ld - h.tdh) * (uint32_t)h.T) + r * (uint32_t)h.tdh +
         g * (uint32_t)(h.T - 1) * (uint32_t)h.tdh + c2;
}

}  // namespace llattn
