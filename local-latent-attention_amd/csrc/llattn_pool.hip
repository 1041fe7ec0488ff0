// Segment pooling of token rows and its broadcast backward, for gfx950.
//
// pool: out[b][n][:] = sum_{t in [n*seg, min((n+1)*seg, T))} x[b][t][:] / divisor
// (reference models.py:159-214 with divisor = real token count; reference
// models.py:216-230 with divisor = seg, the zero-padded mean; divisor 1 folds
// per-token gradients onto latent queries).
//
// HBM-bound: each workgroup reduces one segment over a 32-lane x 16-byte
// column strip (coalesced 512-byte row reads by 8 row groups), then combines
// the row groups in LDS.  The backward is a vectorised broadcast.
#include "llattn_abi.h"
#include "llattn_device.h"

namespace llattn {

struct PoolArgs {
  const void* x; int64_t x_sb, x_st;
  void* out; int64_t o_sb, o_sn;
  int B, T, D, seg, n_seg, divisor, accumulate;
};

__device__ __forceinline__ float seg_scale(int n, const PoolArgs& a) {
  if (a.divisor == LLATTN_DIV_COUNT) return 1.f / (float)(min((n + 1) * a.seg, a.T) - n * a.seg);
  if (a.divisor == LLATTN_DIV_SEG) return 1.f / (float)a.seg;
  return 1.f;
}

template <typename T>
__device__ __forceinline__ void load_vec16(const T* p, float (&v)[Vec16<T>::N]) {
  const uint4 x = ld16(p);
  const T* e = reinterpret_cast<const T*>(&x);
#pragma unroll
  for (int j = 0; j < Vec16<T>::N; ++j) v[j] = to_f<T>(e[j]);
}
template <typename T>
__device__ __forceinline__ void store_vec16(T* p, const float (&v)[Vec16<T>::N]) {
  uint4 x;
  T* e = reinterpret_cast<T*>(&x);
#pragma unroll
  for (int j = 0; j < Vec16<T>::N; ++j) e[j] = from_f<T>(v[j]);
  st16(p, x);
}

template <typename T>
__global__ __launch_bounds__(256) void pool_fwd_kernel(const PoolArgs a) {
  constexpr int V = Vec16<T>::N;
  __shared__ float red[8][32 * V];
  const int n = blockIdx.x % a.n_seg, b = blockIdx.x / a.n_seg;
  const int cthr = threadIdx.x & 31, rg = threadIdx.x >> 5;
  const int col = (blockIdx.y * 32 + cthr) * V;
  const int t0 = n * a.seg, t1 = min(t0 + a.seg, a.T);
  float acc[V];
#pragma unroll
  for (int j = 0; j < V; ++j) acc[j] = 0.f;
  if (col < a.D) {
    const T* xb = static_cast<const T*>(a.x) + b * a.x_sb + col;
    for (int t = t0 + rg; t < t1; t += 8) {
      float v[V];
      load_vec16<T>(xb + (int64_t)t * a.x_st, v);
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] += v[j];
    }
  }
#pragma unroll
  for (int j = 0; j < V; ++j) red[rg][cthr * V + j] = acc[j];
  __syncthreads();
  if (rg == 0 && col < a.D) {
    const float sc = seg_scale(n, a);
    float v[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      float s = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) s += red[k][cthr * V + j];
      v[j] = s * sc;
    }
    store_vec16<T>(static_cast<T*>(a.out) + b * a.o_sb + (int64_t)n * a.o_sn + col, v);
  }
}

// dx[b][t][:] (+)= dpooled[b][t/seg][:] * scale(t/seg).  Here a.x is dpooled
// (rows indexed by segment) and a.out is dx (rows indexed by token).
template <typename T>
__global__ __launch_bounds__(256) void pool_bwd_kernel(const PoolArgs a) {
  constexpr int V = Vec16<T>::N;
  const int cpr = a.D / V;
  const int64_t total = (int64_t)a.B * a.T * cpr;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    const int c = idx % cpr;
    const int64_t bt = idx / cpr;
    const int t = bt % a.T, b = bt / a.T, n = t / a.seg;
    const float sc = seg_scale(n, a);
    float g[V], o[V];
    load_vec16<T>(static_cast<const T*>(a.x) + b * a.x_sb + (int64_t)n * a.x_st + c * V, g);
    T* dp = static_cast<T*>(a.out) + b * a.o_sb + (int64_t)t * a.o_sn + c * V;
    if (a.accumulate) {
      load_vec16<T>(dp, o);
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) o[j] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < V; ++j) o[j] += g[j] * sc;
    store_vec16<T>(dp, o);
  }
}

namespace {
int32_t check_pool(const char* who, const void* x, int64_t x_sb, int64_t x_st, const void* out, int64_t o_sb,
                   int64_t o_sn, int32_t B, int32_t T, int32_t D, int32_t seg, int32_t n_seg, int32_t divisor,
                   int32_t dtype) {
  if (dtype != LLATTN_F32 && dtype != LLATTN_BF16) return fail(LLATTN_ERR_DTYPE, "%s: unknown dtype code %d", who, dtype);
  if (B <= 0 || T <= 0 || D <= 0 || seg <= 0 || n_seg <= 0)
    return fail(LLATTN_ERR_SHAPE, "%s: sizes must be positive (B=%d T=%d D=%d seg=%d n_seg=%d)", who, B, T, D, seg,
                n_seg);
  if ((int64_t)(n_seg - 1) * seg >= T || (int64_t)n_seg * seg < T)
    return fail(LLATTN_ERR_SHAPE, "%s: %d segments of %d tokens do not tile T=%d", who, n_seg, seg, T);
  if (divisor < LLATTN_DIV_COUNT || divisor > LLATTN_DIV_ONE) return fail(LLATTN_ERR_SHAPE, "%s: bad divisor %d", who, divisor);
  const int64_t vec = 16 / elem_size(dtype);
  if (!x || !out || !aligned16(x) || !aligned16(out))
    return fail(LLATTN_ERR_LAYOUT, "%s: pointers must be non-null and 16-byte aligned", who);
  if (D % vec || x_sb % vec || x_st % vec || o_sb % vec || o_sn % vec)
    return fail(LLATTN_ERR_LAYOUT, "%s: D and strides must be multiples of %lld elements", who, (long long)vec);
  return LLATTN_OK;
}
}  // namespace
}  // namespace llattn

using namespace llattn;

extern "C" int32_t llattn_pool_fwd(const void* x, int64_t x_sb, int64_t x_st, void* out, int64_t out_sb,
                                   int64_t out_sn, int32_t B, int32_t T, int32_t D, int32_t seg, int32_t n_seg,
                                   int32_t divisor, int32_t dtype, void* stream) {
  int32_t rc = check_pool("llattn_pool_fwd", x, x_sb, x_st, out, out_sb, out_sn, B, T, D, seg, n_seg, divisor, dtype);
  if (rc) return rc;
  PoolArgs a{x, x_sb, x_st, out, out_sb, out_sn, B, T, D, seg, n_seg, divisor, 0};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int V = 16 / (int)elem_size(dtype);
  const dim3 grid(B * n_seg, (D + 32 * V - 1) / (32 * V));
  if (dtype == LLATTN_F32)
    hipLaunchKernelGGL(pool_fwd_kernel<float>, grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(pool_fwd_kernel<uint16_t>, grid, dim3(256), 0, st, a);
  return check_launch("llattn_pool_fwd");
}

extern "C" int32_t llattn_pool_bwd(const void* dpooled, int64_t dp_sb, int64_t dp_sn, void* dx, int64_t dx_sb,
                                   int64_t dx_st, int32_t B, int32_t T, int32_t D, int32_t seg, int32_t n_seg,
                                   int32_t divisor, int32_t accumulate, int32_t dtype, void* stream) {
  int32_t rc =
      check_pool("llattn_pool_bwd", dpooled, dp_sb, dp_sn, dx, dx_sb, dx_st, B, T, D, seg, n_seg, divisor, dtype);
  if (rc) return rc;
  PoolArgs a{dpooled, dp_sb, dp_sn, dx, dx_sb, dx_st, B, T, D, seg, n_seg, divisor, accumulate ? 1 : 0};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int V = 16 / (int)elem_size(dtype);
  const int64_t total = (int64_t)B * T * (D / V);
  const int blocks = (int)std::min<int64_t>((total + 255) / 256, 8192);
  if (dtype == LLATTN_F32)
    hipLaunchKernelGGL(pool_bwd_kernel<float>, dim3(blocks), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(pool_bwd_kernel<uint16_t>, dim3(blocks), dim3(256), 0, st, a);
  return check_launch("llattn_pool_bwd");
}
