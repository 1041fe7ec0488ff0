// Host-side helpers shared by the entry points: error state and argument checks.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>

#include "llattn.h"

namespace llattn {

// Records a formatted message as the calling thread's last error and returns `code`.
int32_t fail(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the calling thread's last error.
void clear_error();
// Converts a pending launch error into LLATTN_ERR_LAUNCH.
int32_t check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int64_t elem_size(int32_t dtype) { return dtype == LLATTN_F32 ? 4 : 2; }
// smallest padded head dim supported by the compiled kernels (32, 64, 96, 128 or 256), or 0
inline int padded_head_dim(int d) {
  if (d <= 0) return 0;
  if (d <= 32) return 32;
  if (d <= 64) return 64;
  if (d <= 96) return 96;
  if (d <= 128) return 128;
  if (d <= 256) return 256;
  return 0;
}
// Validates a view whose innermost (head-dim) rows are read with 16-byte accesses.
int32_t check_view(const char* name, const llattn_tensor* t, int32_t dtype, bool heads);
int32_t check_shape(const llattn_shape* s);
// workspace bytes of llattn_latent_bwd for a checked shape
size_t latent_workspace_bytes(const llattn_shape* s);

// Split-head storage (llattn_heads_layout) as the kernels address it: divisions by T and dh become
// multiply-high reciprocals (x / d = (umulhi(x, m) + x) >> s, exact for x < 2^31; Granlund and Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994, the 32-bit round-up variant).
struct HeadsMap {
  int T, dh, n, cols;       // cols = n dh; T = 0: plain row-major storage
  uint32_t mt, st, md, sd;  // reciprocals of T and dh
  uint32_t tail;            // element offset of the block of the other columns: rows * cols
  int tail_ld;              // their number per row: ld - cols
  int tdh;                  // 0: that block as packed rows; else as slabs of tdh columns
  uint32_t mtd, std;        // reciprocal of tdh
};
// The reciprocal (m, s) of a divisor 1 <= d < 2^31.
void magic_div(uint32_t d, uint32_t* m, uint32_t* s);
// Checks a split-head layout of a stored matrix of `rows` token rows, `ld` elements apart, whose first
// `width` columns are used, and fills `out` (l NULL or l->T == 0: plain storage, out->T = 0).  `who` names the
// entry point in the error message.
int32_t heads_map(const char* who, const llattn_heads_layout* l, int64_t rows, int64_t ld, int64_t width,
                  HeadsMap* out);

}  // namespace llattn
