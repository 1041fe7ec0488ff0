// Column sums of a bf16 matrix in fp32: out[n] = sum_m x[m][n].  The bias
// gradient of every projection of the block (sum over tokens of the output
// gradient).  HBM-bound: each element is read once with 16-byte loads.
//
// Pass 1: workgroup (column stripe of 128, row block).  Sixteen lanes cover a
// stripe row (eight columns each), so one load instruction of a wave reads four
// whole rows; the 16 row slots of the workgroup (4 waves x 4) are added in LDS
// in a fixed order into one partial row per row block.  Pass 2: out[n] = the
// partial rows added in order.  Deterministic, no atomics.
#include "llattn_abi.h"
#include "llattn_device.h"

namespace llattn {
namespace {

constexpr int kStripe = 128;    // columns per workgroup (16 lanes x 8)
constexpr int kRowBlocks = 64;  // partial rows

__global__ __launch_bounds__(256) void colsum_partial_kernel(const uint16_t* __restrict__ x, int64_t ld, int M, int N,
                                                             int rows_per_block, float* __restrict__ part) {
  __shared__ float red[16][kStripe + 4];
  const int tid = threadIdx.x, slot = tid >> 4, c16 = tid & 15;  // slot: row offset 0..15 within a group of 16 rows
  const int col = blockIdx.x * kStripe + c16 * 8;
  const int r0 = blockIdx.y * rows_per_block, r1 = min(M, r0 + rows_per_block);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  auto add = [&](const uint4 v) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[2 * e] += __uint_as_float(w[e] << 16);
      acc[2 * e + 1] += __uint_as_float(w[e] & 0xffff0000u);
    }
  };
  if (col < N) {
    const uint16_t* p = x + col;
    int rr = r0 + slot;
    for (; rr + 48 < r1; rr += 64) {  // four rows in flight per lane
      uint4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = ld16(p + (int64_t)(rr + 16 * u) * ld);
#pragma unroll
      for (int u = 0; u < 4; ++u) add(v[u]);
    }
    for (; rr < r1; rr += 16) add(ld16(p + (int64_t)rr * ld));
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[slot][c16 * 8 + e] = acc[e];
  __syncthreads();
  if (tid < kStripe) {
    const int c = blockIdx.x * kStripe + tid;
    if (c < N) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) s += red[i][tid];
      part[(int64_t)blockIdx.y * N + c] = s;
    }
  }
}

__global__ __launch_bounds__(256) void colsum_final_kernel(const float* __restrict__ part, int N, int nblk,
                                                           float* __restrict__ out) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  float s = 0.f;
  int i = 0;
  for (; i + 8 <= nblk; i += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = part[(int64_t)(i + u) * N + n];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; i < nblk; ++i) s += part[(int64_t)i * N + n];
  out[n] = s;
}

int row_blocks(int M) { return max(1, min(kRowBlocks, (M + 63) / 64)); }

}  // namespace
}  // namespace llattn

using namespace llattn;

extern "C" size_t llattn_colsum_workspace_size(int32_t M, int32_t N) {
  if (M <= 0 || N <= 0) return 0;
  return (size_t)row_blocks(M) * N * sizeof(float);
}

extern "C" int32_t llattn_colsum(const void* x, int64_t ld, int32_t M, int32_t N, float* out, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  if (M <= 0 || N <= 0) return fail(LLATTN_ERR_SHAPE, "llattn_colsum: sizes must be positive (M=%d N=%d)", M, N);
  if (!x || !out || !aligned16(x) || ld % 8 || N % 8 || ld < N)
    return fail(LLATTN_ERR_LAYOUT, "llattn_colsum: x must be 16-byte aligned with N and ld multiples of 8 (N=%d ld=%lld)",
                N, (long long)ld);
  const size_t need = llattn_colsum_workspace_size(M, N);
  if (!workspace || workspace_bytes < need)
    return fail(LLATTN_ERR_WORKSPACE, "llattn_colsum needs %zu workspace bytes (got %zu)", need, workspace_bytes);
  const int nblk = row_blocks(M);
  const int rows_per_block = (M + nblk - 1) / nblk;
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  hipLaunchKernelGGL(colsum_partial_kernel, dim3((N + kStripe - 1) / kStripe, nblk), dim3(256), 0, st,
                     static_cast<const uint16_t*>(x), ld, M, N, rows_per_block, part);
  hipLaunchKernelGGL(colsum_final_kernel, dim3((N + 255) / 256), dim3(256), 0, st, part, N, nblk, out);
  return check_launch("llattn_colsum");
}
