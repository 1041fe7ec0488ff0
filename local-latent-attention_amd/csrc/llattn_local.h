// Arguments shared by the local-attention kernels (llattn_local.hip) and the
// wide-window backward (llattn_local_wide.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llattn {

struct LocalArgs {
  int B, T, H, Dh, W, bs, q_block, n_qt, gate_hs;
  float scale, scale_log2;
  const void* q; int64_t q_sb, q_st, q_sh;
  const void* k; int64_t k_sb, k_st, k_sh;
  const void* v; int64_t v_sb, v_st, v_sh;
  const void* rem; int64_t r_sb, r_sn, r_sh;
  const float* gl;
  const float* gr;
  void* y; int64_t y_sb, y_st, y_sh;
  void* ol; int64_t o_sb, o_st, o_sh;
  float* lse;  // [B][H][T]
  float* w;    // [B][H][T]
  const void* dy; int64_t dy_sb, dy_st, dy_sh;
  void* dq; int64_t dq_sb, dq_st, dq_sh;
  void* dk; int64_t dk_sb, dk_st, dk_sh;
  void* dv; int64_t dv_sb, dv_st, dv_sh;
  void* dr; int64_t dr_sb, dr_st, dr_sh;
  void* dO;      // workspace [B][T][H][Dh], storage type
  float* Dsum;   // workspace [B][H][T]
  float* gpart;  // workspace [H][3][Dh][rows]: gate_l, gate_r and dremote column partial sums
};

// Row strides below 2^24 elements and (batch, head) slabs of T rows below 2^30
// elements, so that kernels may address a slab with 32-bit byte offsets.
bool strides_fit_32bit(const LocalArgs& a);

// The wide-window backward (llattn_local_wide.hip) takes bf16 calls with
// windows above 64 and padded head dims up to 128.
bool wide_bwd(const LocalArgs& a, int dtype, int dhp);
// Its gate partial rows: one per (batch, 128-query group).
int wide_gate_rows(const LocalArgs& a);
// Launches its two kernels (query side, then key side).
void launch_bwd_wide(const LocalArgs& a, int dhp, hipStream_t stream);

// The forward on 32x32x16 products (llattn_local_wide.hip) takes bf16 calls of
// any window with padded head dims up to 128.
bool fwd32(const LocalArgs& a, int dtype, int dhp);
void launch_fwd32(const LocalArgs& a, int dhp, hipStream_t stream);

}  // namespace llattn
