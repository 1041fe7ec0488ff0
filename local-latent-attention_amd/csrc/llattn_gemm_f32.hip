// fp32 projection GEMM for gfx950: C = A Bᵀ (+ bias) (+ C) with fp32 operands and fp32 accumulation on
// v_mfma_f32_16x16x4_f32, the fp32 counterpart of llattn_gemm for the fp32 module (the reference's
// nn.Linear products in fp32, models.py:80-84, 315, 333-353, 395, 462, and their autograd).
//
// Same descriptor and operand layouts as llattn_gemm: A(m, k) is A[m * lda + k] (a_trans = 0) or
// A[k * lda + m] (a_trans = 1); B(n, k) is B[n * ldb + k] (b_trans = 0) or B[k * ldb + n] (b_trans = 1).
// One 256-thread workgroup per 64 x 64 output tile, four waves of 32 x 32 (2 x 2 MFMA blocks of 16 x 16).
// K advances in 16-wide steps: each thread loads four elements of the A tile and four of the B tile
// (16-byte loads along the contiguous dimension where it is in range and aligned), the tile is stored
// k-major in LDS, and every wave runs four k-substeps of 4.  Rows, columns and k past the matrix read zero.
// With a_rowsum, the workgroups of the first tile column also add the A tile over k into one fp32 sum per
// row (in k order), the bias gradient of a weight-gradient product dyᵀ x.  Deterministic: every output has
// one writer and a fixed summation order.  A correctness path for fp32 models, not a tuned one.
#include "llattn_abi.h"
#include "llattn_device.h"

namespace llattn {
namespace {

constexpr int FT = 64, FK = 16, FP = FT + 4;  // tile, k step, padded LDS row (floats)

struct GemmF32Args {
  int M, N, K, a_trans, b_trans, accumulate;
  const float* A;
  int64_t lda;
  const float* B;
  int64_t ldb;
  float* C;
  int64_t ldc;
  const float* bias;
  float* rowsum;
};

// 4 elements of a 64 x 16 operand tile into the k-major LDS tile s[k][o] (o: row of the product operand).
// k-contiguous storage: thread t takes row o = t / 4 and k = 4 (t % 4) .. + 3; m/n-contiguous storage:
// k = t / 16 and o = 4 (t % 16) .. + 3.  Out-of-range elements are zero.
__device__ __forceinline__ void load_tile(const float* __restrict__ p, int64_t ld, bool kcontig, int o0, int k0,
                                          int O, int K, int t, float (*s)[FP]) {
  float v[4];
  int o, k;
  if (kcontig) {
    o = t >> 2;
    k = 4 * (t & 3);
    const int go = o0 + o, gk = k0 + k;
    const float* q = p + (int64_t)go * ld + gk;
    if (go < O && gk + 3 < K && ((uintptr_t)q & 15) == 0) {
      const float4 x = *reinterpret_cast<const float4*>(q);
      v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (go < O && gk + e < K) ? q[e] : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) s[k + e][o] = v[e];
  } else {
    k = t >> 4;
    o = 4 * (t & 15);
    const int go = o0 + o, gk = k0 + k;
    const float* q = p + (int64_t)gk * ld + go;
    if (gk < K && go + 3 < O && ((uintptr_t)q & 15) == 0) {
      const float4 x = *reinterpret_cast<const float4*>(q);
      v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (gk < K && go + e < O) ? q[e] : 0.f;
    }
    *reinterpret_cast<float4*>(&s[k][o]) = make_float4(v[0], v[1], v[2], v[3]);
  }
}

__global__ __launch_bounds__(256) void gemm_f32_kernel(const GemmF32Args a) {
  __shared__ __align__(16) float As[FK][FP];
  __shared__ __align__(16) float Bs[FK][FP];
  const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
  const int wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
  const int tiles_n = (a.N + FT - 1) / FT;
  const int m0 = (blockIdx.x / tiles_n) * FT, n0 = (blockIdx.x % tiles_n) * FT;
  const bool rs = a.rowsum != nullptr && n0 == 0;  // workgroup-uniform
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float rsum = 0.f;  // rs: thread t < 64 sums row m0 + t of A over k
  for (int k0 = 0; k0 < a.K; k0 += FK) {
    load_tile(a.A, a.lda, !a.a_trans, m0, k0, a.M, a.K, tid, As);
    load_tile(a.B, a.ldb, !a.b_trans, n0, k0, a.N, a.K, tid, Bs);
    __syncthreads();
    if (rs && tid < FT) {
#pragma unroll
      for (int k = 0; k < FK; ++k) rsum += As[k][tid];
    }
#pragma unroll
    for (int kk = 0; kk < FK; kk += 4) {
      // A operand: lane (r, g) supplies A[m = r][k = g]; B operand: B[n = r][k = g]
      float av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) av[i] = As[kk + g][wm * 32 + 16 * i + r];
#pragma unroll
      for (int j = 0; j < 2; ++j) bv[j] = Bs[kk + g][wn * 32 + 16 * j + r];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
  // lane (r, g) holds C[m = 16 i + 4 g + e][n = 16 j + r] of the wave's 32 x 32 block
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn * 32 + 16 * j + r;
      if (n >= a.N) continue;
      const float b = a.bias ? a.bias[n] : 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + wm * 32 + 16 * i + 4 * g + e;
        if (m >= a.M) continue;
        float* c = a.C + (int64_t)m * a.ldc + n;
        const float v = acc[i][j][e] + b;
        *c = a.accumulate ? *c + v : v;
      }
    }
  if (rs && tid < FT && m0 + tid < a.M) a.rowsum[m0 + tid] = rsum;
}

}  // namespace
}  // namespace llattn

using namespace llattn;

extern "C" int32_t llattn_gemm_f32(const llattn_gemm_desc* d, void* stream) {
  if (!d) return fail(LLATTN_ERR_SHAPE, "llattn_gemm_f32: null descriptor");
  if (d->M <= 0 || d->N <= 0 || d->K <= 0)
    return fail(LLATTN_ERR_SHAPE, "llattn_gemm_f32: sizes must be positive (M=%d N=%d K=%d)", d->M, d->N, d->K);
  if (d->c_dtype != LLATTN_F32)
    return fail(LLATTN_ERR_DTYPE, "llattn_gemm_f32: fp32 C only (c_dtype %d)", d->c_dtype);
  if (d->split_k > 1 || d->rowadd[0].ptr || d->rowadd[1].ptr || d->act != LLATTN_ACT_NONE || d->c_heads.T != 0)
    return fail(LLATTN_ERR_UNSUPPORTED, "llattn_gemm_f32: no K split, row addends, activation or split-head C");
  if (!d->A || !d->B || !d->C || (uintptr_t)d->A % 4 || (uintptr_t)d->B % 4 || (uintptr_t)d->C % 4 ||
      (d->bias && (uintptr_t)d->bias % 4) || (d->a_rowsum && (uintptr_t)d->a_rowsum % 4))
    return fail(LLATTN_ERR_LAYOUT, "llattn_gemm_f32: operands must be non-null and 4-byte aligned");
  if (d->lda < (d->a_trans ? d->M : d->K) || d->ldb < (d->b_trans ? d->N : d->K) || d->ldc < d->N)
    return fail(LLATTN_ERR_LAYOUT, "llattn_gemm_f32: leading dimensions smaller than the rows they hold");
  const int64_t tiles = (int64_t)((d->M + FT - 1) / FT) * ((d->N + FT - 1) / FT);
  if (tiles > 0x7fffffff) return fail(LLATTN_ERR_UNSUPPORTED, "llattn_gemm_f32: too many output tiles");
  GemmF32Args a{};
  a.M = d->M; a.N = d->N; a.K = d->K;
  a.a_trans = d->a_trans; a.b_trans = d->b_trans; a.accumulate = d->accumulate;
  a.A = static_cast<const float*>(d->A); a.lda = d->lda;
  a.B = static_cast<const float*>(d->B); a.ldb = d->ldb;
  a.C = static_cast<float*>(d->C); a.ldc = d->ldc;
  a.bias = d->bias;
  a.rowsum = d->a_rowsum;
  hipLaunchKernelGGL(gemm_f32_kernel, dim3((unsigned)tiles), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("llattn_gemm_f32");
}
