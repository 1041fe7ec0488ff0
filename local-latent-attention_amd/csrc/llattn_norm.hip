// RMSNorm of the blocks' residual stream (reference models.py:40-47, F.rms_norm over the last dim):
//   y[m][d] = x[m][d] * rstd[m] * w[d],   rstd[m] = 1 / sqrt(mean_d x[m][d]^2 + eps)
// and its backward
//   xh = x * rstd,  g = dy * w
//   dx = rstd * (g - xh * mean_d(g * xh)),   dw[d] = sum_m dy[m][d] * xh[m][d]
//
// HBM-bound.  One wave per row: lane l holds the 4-element chunks l, l+64, ... of the row in
// registers (16-byte fp32 / 8-byte bf16 loads), so every element is read once and written once;
// the row sums are wave reductions.  The forward writes y straight in the consumer's dtype (bf16
// under autocast: the projections that read it are bf16), which removes the separate cast.
// The backward runs a fixed grid of waves over contiguous row ranges; each lane keeps its
// columns' dw partial sums in registers, the workgroup's four waves are added in LDS, and a second
// kernel adds the per-workgroup rows in a fixed order (deterministic, no atomics).
#include "llattn_abi.h"
#include "llattn_device.h"

namespace llattn {
namespace {

constexpr int kBwdBlocks = 512;  // workgroups of the backward (two per CU); dw partial rows

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <typename T>
__device__ __forceinline__ void ld4(const T* p, float o[4]) {
  if constexpr (std::is_same_v<T, float>) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  } else {
    unpack_bf16x4(*reinterpret_cast<const uint2*>(p), o);
  }
}

template <typename T>
__device__ __forceinline__ void st4(T* p, const float v[4]) {
  if constexpr (std::is_same_v<T, float>) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
  }
}

// NCH: 4-element chunks per lane (D <= 256 NCH)
template <typename XT, typename YT, int NCH>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const XT* x, int64_t ldx,
                                                          const float* __restrict__ w, int M, int D, float eps,
                                                          YT* __restrict__ y, int64_t ldy, float* __restrict__ rstd,
                                                          const void* res, int r_bf16, int64_t ldr, float* xo,
                                                          int64_t ldxo) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;  // wave-uniform
  const int nq = D >> 2;
  const XT* xr = x + (int64_t)row * ldx;
  float v[NCH][4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane + 64 * i;
    if (c < nq) {
      ld4(xr + 4 * c, v[i]);
      if (res) {  // residual add first (fp32, as x + res promotes): the normalised rows are those of the sum
        float rv[4];
        if (r_bf16) ld4(static_cast<const uint16_t*>(res) + (int64_t)row * ldr + 4 * c, rv);
        else ld4(static_cast<const float*>(res) + (int64_t)row * ldr + 4 * c, rv);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[i][e] += rv[e];
        st4(xo + (int64_t)row * ldxo + 4 * c, v[i]);
      }
    } else {
      v[i][0] = v[i][1] = v[i][2] = v[i][3] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += v[i][e] * v[i][e];
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)D + eps);
  if (lane == 0) rstd[row] = r;
  YT* yr = y + (int64_t)row * ldy;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane + 64 * i;
    if (c < nq) {
      const float4 w4 = *reinterpret_cast<const float4*>(w + 4 * c);
      const float o[4] = {v[i][0] * r * w4.x, v[i][1] * r * w4.y, v[i][2] * r * w4.z, v[i][3] * r * w4.w};
      st4(yr + 4 * c, o);
    }
  }
}

template <typename XT, typename DYT, int NCH>
__global__ __launch_bounds__(256, NCH <= 6 ? 2 : 1) void rmsnorm_bwd_kernel(const DYT* __restrict__ dy, int64_t lddy,
                                                          const XT* __restrict__ x, int64_t ldx,
                                                          const float* __restrict__ rstd,
                                                          const float* __restrict__ w, int M, int D,
                                                          XT* __restrict__ dx, int64_t lddx,
                                                          float* __restrict__ part, const XT* dres, int64_t lddres) {
  extern __shared__ float red[];  // [4][D]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nq = D >> 2;
  const int nw = gridDim.x * 4, gw = blockIdx.x * 4 + wave;
  const int per = (M + nw - 1) / nw;
  const int r0 = min(M, gw * per), r1 = min(M, r0 + per);
  // Chunks past the row read a valid chunk (0) and are then zeroed by a select: every array element is
  // written unconditionally, so the arrays stay in registers (element writes under a branch made the
  // compiler keep them in scratch memory).
  float wv[NCH][4], dw[NCH][4];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane + 64 * i;
    const bool ok = c < nq;
    const float4 w4 = *reinterpret_cast<const float4*>(w + 4 * (ok ? c : 0));
    wv[i][0] = ok ? w4.x : 0.f;
    wv[i][1] = ok ? w4.y : 0.f;
    wv[i][2] = ok ? w4.z : 0.f;
    wv[i][3] = ok ? w4.w : 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) dw[i][e] = 0.f;
  }
  const float inv_d = 1.0f / (float)D;
  // row data of the next row -- x, dy and rstd -- is loaded before the current row is computed (two
  // register sets), so no load issued while a row is computed is waited for by that row
  auto load_row = [&](int row, float (&xv)[NCH][4], float (&dv)[NCH][4], float& rs) {
    const XT* xr = x + (int64_t)row * ldx;
    const DYT* dr = dy + (int64_t)row * lddy;
    rs = rstd[row];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane + 64 * i;
      const bool ok = c < nq;
      float xt[4], dt[4];
      ld4(xr + 4 * (ok ? c : 0), xt);
      ld4(dr + 4 * (ok ? c : 0), dt);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xv[i][e] = ok ? xt[e] : 0.f;
        dv[i][e] = ok ? dt[e] : 0.f;
      }
    }
  };
  const int64_t ldo = lddx, ldr = lddres;
  // xh = x * rstd and g = dy * w are formed twice (for the row dot product, then for dx) rather than kept
  auto do_row = [&](int row, const float (&xv)[NCH][4], const float (&dv)[NCH][4], const float r) {
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) dot += (dv[i][e] * wv[i][e]) * (xv[i][e] * r);
    const float mdot = wave_sum(dot) * inv_d;
    XT* o = dx + (int64_t)row * ldo;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane + 64 * i;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float xh = xv[i][e] * r;
        v[e] = r * (dv[i][e] * wv[i][e] - xh * mdot);
        dw[i][e] += dv[i][e] * xh;
      }
      if (c < nq) {
        if (dres) {  // the gradient that reaches the normalised rows' input through the residual path
          float g[4];
          ld4(dres + (int64_t)row * ldr + 4 * c, g);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] += g[e];
        }
        st4(o + 4 * c, v);
      }
    }
  };
  float xa[NCH][4], da[NCH][4], ra = 0.f;
  if constexpr (NCH <= 8) {  // two register sets: the next row loads while this one is computed
    float xb[NCH][4], db[NCH][4], rb = 0.f;
    if (r0 < r1) load_row(r0, xa, da, ra);
    for (int row = r0; row < r1; row += 2) {
      if (row + 1 < r1) load_row(row + 1, xb, db, rb);
      do_row(row, xa, da, ra);
      if (row + 1 >= r1) break;
      if (row + 2 < r1) load_row(row + 2, xa, da, ra);
      do_row(row + 1, xb, db, rb);
    }
  } else {
    for (int row = r0; row < r1; ++row) {
      load_row(row, xa, da, ra);
      do_row(row, xa, da, ra);
    }
  }
  // the workgroup's four waves, added in wave order
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane + 64 * i;
    if (c < nq) {
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wave * D + 4 * c + e] = dw[i][e];
    }
  }
  __syncthreads();
  for (int col = threadIdx.x; col < D; col += 256)
    part[(int64_t)blockIdx.x * D + col] = ((red[col] + red[D + col]) + red[2 * D + col]) + red[3 * D + col];
}

// dw[d] = sum over the partial rows in order.  Workgroup: 64 columns x 4 row groups; group q adds rows
// q, q+4, ... (16 loads in flight per thread); the four group sums are added in group order.
__global__ __launch_bounds__(256) void rmsnorm_dw_kernel(const float* __restrict__ part, int nrows, int D,
                                                         float* __restrict__ dw) {
  __shared__ float red[4][64];
  const int cl = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + cl;
  float s = 0.f;
  if (col < D) {
    int i = q;
    for (; i + 4 * 15 < nrows; i += 4 * 16) {
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = part[(int64_t)(i + 4 * u) * D + col];
#pragma unroll
      for (int u = 0; u < 16; ++u) s += v[u];
    }
    for (; i < nrows; i += 4) s += part[(int64_t)i * D + col];
  }
  red[q][cl] = s;
  __syncthreads();
  if (q == 0 && col < D) dw[col] = ((red[0][cl] + red[1][cl]) + red[2][cl]) + red[3][cl];
}

int chunks_for(int D) {  // 4-element chunks per lane, rounded up to a compiled count
  const int n = (D / 4 + 63) / 64;
  return n <= 2 ? 2 : n <= 4 ? 4 : n <= 6 ? 6 : n <= 8 ? 8 : n <= 12 ? 12 : n <= 16 ? 16 : 0;
}

template <typename XT, typename YT>
void launch_fwd(int nch, const void* x, int64_t ldx, const float* w, int M, int D, float eps, void* y, int64_t ldy,
                float* rstd, const void* r, int r_bf16, int64_t ldr, float* xo, int64_t ldxo, hipStream_t st) {
  const dim3 grid((M + 3) / 4), block(256);
  const XT* xp = static_cast<const XT*>(x);
  YT* yp = static_cast<YT*>(y);
  switch (nch) {
    case 2: hipLaunchKernelGGL((rmsnorm_fwd_kernel<XT, YT, 2>), grid, block, 0, st, xp, ldx, w, M, D, eps, yp, ldy, rstd, r, r_bf16, ldr, xo, ldxo); break;
    case 4: hipLaunchKernelGGL((rmsnorm_fwd_kernel<XT, YT, 4>), grid, block, 0, st, xp, ldx, w, M, D, eps, yp, ldy, rstd, r, r_bf16, ldr, xo, ldxo); break;
    case 6: hipLaunchKernelGGL((rmsnorm_fwd_kernel<XT, YT, 6>), grid, block, 0, st, xp, ldx, w, M, D, eps, yp, ldy, rstd, r, r_bf16, ldr, xo, ldxo); break;
    case 8: hipLaunchKernelGGL((rmsnorm_fwd_kernel<XT, YT, 8>), grid, block, 0, st, xp, ldx, w, M, D, eps, yp, ldy, rstd, r, r_bf16, ldr, xo, ldxo); break;
    case 12: hipLaunchKernelGGL((rmsnorm_fwd_kernel<XT, YT, 12>), grid, block, 0, st, xp, ldx, w, M, D, eps, yp, ldy, rstd, r, r_bf16, ldr, xo, ldxo); break;
    default: hipLaunchKernelGGL((rmsnorm_fwd_kernel<XT, YT, 16>), grid, block, 0, st, xp, ldx, w, M, D, eps, yp, ldy, rstd, r, r_bf16, ldr, xo, ldxo); break;
  }
}

template <typename XT, typename DYT>
void launch_bwd(int nch, int nblk, const void* dy, int64_t lddy, const void* x, int64_t ldx, const float* rstd,
                const float* w, int M, int D, void* dx, int64_t lddx, float* part, const void* dres, int64_t lddres,
                hipStream_t st) {
  const dim3 grid(nblk), block(256);
  const size_t lds = (size_t)4 * D * sizeof(float);
  const DYT* dyp = static_cast<const DYT*>(dy);
  const XT* xp = static_cast<const XT*>(x);
  XT* dxp = static_cast<XT*>(dx);
  switch (nch) {
    case 2: hipLaunchKernelGGL((rmsnorm_bwd_kernel<XT, DYT, 2>), grid, block, lds, st, dyp, lddy, xp, ldx, rstd, w, M, D, dxp, lddx, part, static_cast<const XT*>(dres), lddres); break;
    case 4: hipLaunchKernelGGL((rmsnorm_bwd_kernel<XT, DYT, 4>), grid, block, lds, st, dyp, lddy, xp, ldx, rstd, w, M, D, dxp, lddx, part, static_cast<const XT*>(dres), lddres); break;
    case 6: hipLaunchKernelGGL((rmsnorm_bwd_kernel<XT, DYT, 6>), grid, block, lds, st, dyp, lddy, xp, ldx, rstd, w, M, D, dxp, lddx, part, static_cast<const XT*>(dres), lddres); break;
    case 8: hipLaunchKernelGGL((rmsnorm_bwd_kernel<XT, DYT, 8>), grid, block, lds, st, dyp, lddy, xp, ldx, rstd, w, M, D, dxp, lddx, part, static_cast<const XT*>(dres), lddres); break;
    case 12: hipLaunchKernelGGL((rmsnorm_bwd_kernel<XT, DYT, 12>), grid, block, lds, st, dyp, lddy, xp, ldx, rstd, w, M, D, dxp, lddx, part, static_cast<const XT*>(dres), lddres); break;
    default: hipLaunchKernelGGL((rmsnorm_bwd_kernel<XT, DYT, 16>), grid, block, lds, st, dyp, lddy, xp, ldx, rstd, w, M, D, dxp, lddx, part, static_cast<const XT*>(dres), lddres); break;
  }
}

int32_t check_rows(const char* what, const char* name, const void* p, int64_t ld, int32_t dtype, int32_t D) {
  if (!p) return fail(LLATTN_ERR_LAYOUT, "%s: %s is null", what, name);
  if (dtype != LLATTN_F32 && dtype != LLATTN_BF16) return fail(LLATTN_ERR_DTYPE, "%s: unknown dtype %d of %s", what, dtype, name);
  const int64_t align = dtype == LLATTN_F32 ? 16 : 8;
  if ((reinterpret_cast<uintptr_t>(p) % align) || (ld * elem_size(dtype)) % align || ld < D)
    return fail(LLATTN_ERR_LAYOUT, "%s: rows of %s must be %lld-byte aligned with ld >= D (ld=%lld)", what, name,
                (long long)align, (long long)ld);
  return LLATTN_OK;
}

int32_t check_dims(const char* what, int32_t M, int32_t D) {
  if (M <= 0 || D <= 0) return fail(LLATTN_ERR_SHAPE, "%s: sizes must be positive (M=%d D=%d)", what, M, D);
  if (D % 4 || !chunks_for(D))
    return fail(LLATTN_ERR_UNSUPPORTED, "%s: D=%d must be a multiple of 4 and at most 4096", what, D);
  return LLATTN_OK;
}

}  // namespace
}  // namespace llattn

using namespace llattn;

extern "C" int32_t llattn_rmsnorm_fwd(const void* x, int32_t x_dtype, int64_t ldx, const float* weight, int32_t M,
                                      int32_t D, float eps, void* y, int32_t y_dtype, int64_t ldy, float* rstd,
                                      const void* res, int32_t res_dtype, int64_t ldres, float* xsum, int64_t ldxsum,
                                      void* stream) {
  const char* what = "llattn_rmsnorm_fwd";
  int32_t rc;
  if ((rc = check_dims(what, M, D)) || (rc = check_rows(what, "x", x, ldx, x_dtype, D)) ||
      (rc = check_rows(what, "y", y, ldy, y_dtype, D)))
    return rc;
  if (res) {
    if (x_dtype != LLATTN_F32)
      return fail(LLATTN_ERR_DTYPE, "%s: a residual addend needs fp32 x (the sum is kept in fp32)", what);
    if ((rc = check_rows(what, "res", res, ldres, res_dtype, D)) ||
        (rc = check_rows(what, "xsum", xsum, ldxsum, LLATTN_F32, D)))
      return rc;
  }
  if (!weight || !aligned16(weight) || !rstd)
    return fail(LLATTN_ERR_LAYOUT, "%s: weight (16-byte aligned fp32 [D]) and rstd (fp32 [M]) are required", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nch = chunks_for(D);
  const int rb = res && res_dtype == LLATTN_BF16;
  if (x_dtype == LLATTN_F32 && y_dtype == LLATTN_F32) launch_fwd<float, float>(nch, x, ldx, weight, M, D, eps, y, ldy, rstd, res, rb, ldres, xsum, ldxsum, st);
  else if (x_dtype == LLATTN_F32) launch_fwd<float, uint16_t>(nch, x, ldx, weight, M, D, eps, y, ldy, rstd, res, rb, ldres, xsum, ldxsum, st);
  else if (y_dtype == LLATTN_F32) launch_fwd<uint16_t, float>(nch, x, ldx, weight, M, D, eps, y, ldy, rstd, nullptr, 0, 0, nullptr, 0, st);
  else launch_fwd<uint16_t, uint16_t>(nch, x, ldx, weight, M, D, eps, y, ldy, rstd, nullptr, 0, 0, nullptr, 0, st);
  return check_launch(what);
}

extern "C" size_t llattn_rmsnorm_workspace_size(int32_t M, int32_t D) {
  if (M <= 0 || D <= 0) return 0;
  return (size_t)kBwdBlocks * D * sizeof(float);
}

extern "C" int32_t llattn_rmsnorm_bwd(const void* dy, int32_t dy_dtype, int64_t lddy, const void* x, int32_t x_dtype,
                                      int64_t ldx, const float* rstd, const float* weight, int32_t M, int32_t D,
                                      void* dx, int64_t lddx, float* dweight, const void* dres, int64_t lddres,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "llattn_rmsnorm_bwd";
  int32_t rc;
  if ((rc = check_dims(what, M, D)) || (rc = check_rows(what, "dy", dy, lddy, dy_dtype, D)) ||
      (rc = check_rows(what, "x", x, ldx, x_dtype, D)) || (rc = check_rows(what, "dx", dx, lddx, x_dtype, D)))
    return rc;
  if (dres && (rc = check_rows(what, "dres", dres, lddres, x_dtype, D))) return rc;
  if (!weight || !aligned16(weight) || !rstd || !dweight)
    return fail(LLATTN_ERR_LAYOUT, "%s: weight (16-byte aligned fp32 [D]), rstd and dweight are required", what);
  const size_t need = llattn_rmsnorm_workspace_size(M, D);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return fail(LLATTN_ERR_WORKSPACE, "%s needs %zu workspace bytes (got %zu)", what, need, workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nch = chunks_for(D);
  float* part = static_cast<float*>(workspace);
  if (x_dtype == LLATTN_F32 && dy_dtype == LLATTN_F32) launch_bwd<float, float>(nch, kBwdBlocks, dy, lddy, x, ldx, rstd, weight, M, D, dx, lddx, part, dres, lddres, st);
  else if (x_dtype == LLATTN_F32) launch_bwd<float, uint16_t>(nch, kBwdBlocks, dy, lddy, x, ldx, rstd, weight, M, D, dx, lddx, part, dres, lddres, st);
  else if (dy_dtype == LLATTN_F32) launch_bwd<uint16_t, float>(nch, kBwdBlocks, dy, lddy, x, ldx, rstd, weight, M, D, dx, lddx, part, dres, lddres, st);
  else launch_bwd<uint16_t, uint16_t>(nch, kBwdBlocks, dy, lddy, x, ldx, rstd, weight, M, D, dx, lddx, part, dres, lddres, st);
  hipLaunchKernelGGL(rmsnorm_dw_kernel, dim3((D + 63) / 64), dim3(256), 0, st, part, kBwdBlocks, D, dweight);
  return check_launch(what);
}
