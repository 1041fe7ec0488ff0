// Entry points that launch nothing (version, errors, workspace sizes) and the
// argument checks every launcher runs before touching the device.
#include "llattn_abi.h"

#include <cstdio>
#include <cstring>

namespace llattn {

namespace {
thread_local char g_last_error[512] = {0};
}

int32_t fail(int32_t code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = 0; }

int32_t check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LLATTN_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return LLATTN_OK;
}

int32_t check_view(const char* name, const llattn_tensor* t, int32_t dtype, bool heads) {
  if (t == nullptr || t->ptr == nullptr) return fail(LLATTN_ERR_LAYOUT, "%s: null tensor", name);
  const int64_t vec = 16 / elem_size(dtype);
  if (!aligned16(t->ptr)) return fail(LLATTN_ERR_LAYOUT, "%s: base pointer is not 16-byte aligned", name);
  if (t->sb % vec || t->sn % vec || (heads && t->sh % vec))
    return fail(LLATTN_ERR_LAYOUT, "%s: strides (%lld, %lld, %lld) must be multiples of %lld elements", name,
                (long long)t->sb, (long long)t->sn, (long long)t->sh, (long long)vec);
  return LLATTN_OK;
}

int32_t check_shape(const llattn_shape* s) {
  if (s == nullptr) return fail(LLATTN_ERR_SHAPE, "null shape");
  if (s->dtype != LLATTN_F32 && s->dtype != LLATTN_BF16) return fail(LLATTN_ERR_DTYPE, "unknown dtype code %d", s->dtype);
  if (s->B <= 0 || s->T <= 0 || s->H <= 0 || s->Dh <= 0 || s->Lh <= 0 || s->Ldh <= 0)
    return fail(LLATTN_ERR_SHAPE, "sizes must be positive (B=%d T=%d H=%d Dh=%d Lh=%d Ldh=%d)", s->B, s->T, s->H,
                s->Dh, s->Lh, s->Ldh);
  if (s->window <= 0) return fail(LLATTN_ERR_SHAPE, "local_window must be positive (got %d)", s->window);
  if (s->block <= 0 || s->block > s->T)
    return fail(LLATTN_ERR_SHAPE, "local block size %d outside [1, T=%d]", s->block, s->T);
  if (s->chunk <= 0 || s->n_chunks <= 0 || (int64_t)(s->n_chunks - 1) * s->chunk >= s->T ||
      (int64_t)s->n_chunks * s->chunk < s->T)
    return fail(LLATTN_ERR_SHAPE, "latent chunk %d x %d chunks does not tile T=%d", s->chunk, s->n_chunks, s->T);
  if (s->q_block <= 0 || s->n_q <= 0 || (int64_t)(s->n_q - 1) * s->q_block >= s->T ||
      (int64_t)s->n_q * s->q_block < s->T)
    return fail(LLATTN_ERR_SHAPE, "latent query block %d x %d queries does not tile T=%d", s->q_block, s->n_q, s->T);
  const int vec = s->dtype == LLATTN_F32 ? 4 : 8, dmax = s->dtype == LLATTN_F32 ? 128 : 256;
  if (s->Dh % vec || padded_head_dim(s->Dh) == 0 || s->Dh > dmax)
    return fail(LLATTN_ERR_UNSUPPORTED, "head_dim %d unsupported (needs a multiple of %d, at most %d)", s->Dh, vec,
                dmax);
  if (s->Ldh % vec || padded_head_dim(s->Ldh) == 0 || s->Ldh > dmax)
    return fail(LLATTN_ERR_UNSUPPORTED, "latent head_dim %d unsupported (needs a multiple of %d, at most %d)", s->Ldh,
                vec, dmax);
  return LLATTN_OK;
}

void magic_div(uint32_t d, uint32_t* m, uint32_t* s) {
  uint32_t sh = 0;
  while ((uint64_t(1) << sh) < d) ++sh;
  *s = sh;
  *m = (uint32_t)((((uint64_t(1) << sh) - d) << 32) / d + 1);
}

int32_t heads_map(const char* who, const llattn_heads_layout* l, int64_t rows, int64_t ld, int64_t width,
                  HeadsMap* out) {
  *out = HeadsMap{};
  if (l == nullptr || l->T == 0) return LLATTN_OK;
  if (l->T < 0 || l->dh <= 0 || l->n <= 0 || l->dh % 8 || rows % l->T)
    return fail(LLATTN_ERR_LAYOUT, "%s: split-head layout T=%d dh=%d n=%d: needs T, n > 0, dh a positive multiple of "
                "8 and whole sequences of T rows (rows=%lld)", who, l->T, l->dh, l->n, (long long)rows);
  const int64_t cols = (int64_t)l->n * l->dh;
  if (cols > width || width > ld || ld % 8)
    return fail(LLATTN_ERR_LAYOUT, "%s: split-head layout of %lld head columns in a matrix of width %lld, ld %lld",
                who, (long long)cols, (long long)width, (long long)ld);
  if (rows * ld * 2 >= (int64_t(1) << 31))
    return fail(LLATTN_ERR_UNSUPPORTED, "%s: a split-head matrix must be below 2 GiB (%lld x %lld)", who,
                (long long)rows, (long long)ld);
  out->T = l->T;
  out->dh = l->dh;
  out->n = l->n;
  out->cols = (int)cols;
  magic_div((uint32_t)l->T, &out->mt, &out->st);
  magic_div((uint32_t)l->dh, &out->md, &out->sd);
  out->tail = (uint32_t)(rows * cols);
  out->tail_ld = (int)(ld - cols);
  if (l->tail_dh != 0) {
    if (l->tail_dh < 0 || l->tail_dh % 8 || (ld - cols) % l->tail_dh)
      return fail(LLATTN_ERR_LAYOUT, "%s: split-head tail slabs of %d columns: needs a positive multiple of 8 that "
                  "divides the %lld columns past the heads (ld %lld)", who, l->tail_dh, (long long)(ld - cols),
                  (long long)ld);
    out->tdh = l->tail_dh;
    magic_div((uint32_t)l->tail_dh, &out->mtd, &out->std);
  }
  return LLATTN_OK;
}

}  // namespace llattn

using namespace llattn;

extern "C" {

int32_t llattn_abi_version(void) { return LLATTN_ABI_VERSION; }

const char* llattn_last_error(void) { return g_last_error; }

// Local backward workspace: dO_local [B][T][H][Dh] (storage type), row sums
// D [B][H][T] fp32 and gate partials [H][2][Dh][B*n_qtiles] fp32.
// Latent backward workspace: D [B][Lh][n_q] fp32 and per-segment dgk/dgv partials
// [B][Lh][n_segments][16*ceil(n_chunks/16)][2][Ldh] fp32 (see llattn_latent.hip).
size_t llattn_workspace_size(const llattn_shape* s, int32_t kind) {
  if (check_shape(s) != LLATTN_OK) return 0;
  const size_t B = s->B, T = s->T, H = s->H, Dh = s->Dh;
  auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
  if (kind == LLATTN_WS_LOCAL_BWD) {
    const size_t nqt = (T + 63) / 64;
    return up(B * T * H * Dh * elem_size(s->dtype)) + up(B * H * T * 4) + up(B * H * nqt * 3 * Dh * 4);
  }
  if (kind == LLATTN_WS_LATENT_BWD) return latent_workspace_bytes(s);
  fail(LLATTN_ERR_SHAPE, "unknown workspace kind %d", kind);
  return 0;
}

}  // extern "C"
