// fp32 -> bf16 (or fp32 -> fp32) copies of several arrays in one launch: the weight casts that bf16
// autocast performs once per forward for every nn.Linear of the block, and the concatenated biases
// of projections that share one GEMM.  HBM-bound; one pass over each array.
//
// The launch covers the concatenation of all segments in chunks of 8 elements (32 bytes read); each
// thread finds its segment by a scan over the (at most LLATTN_CAST_MAX_SEGS) segment starts.  Segments whose
// source and destination are 16-byte aligned move with 16-byte loads and stores, others element by element.
// Conversion rounds to nearest even, as a torch .to(torch.bfloat16) does.
#include "llattn_abi.h"
#include "llattn_device.h"

namespace llattn {
namespace {

struct CastArgs {
  const float* src[LLATTN_CAST_MAX_SEGS];
  void* dst[LLATTN_CAST_MAX_SEGS];
  int64_t start[LLATTN_CAST_MAX_SEGS + 1];  // chunk index where segment i begins
  int64_t n[LLATTN_CAST_MAX_SEGS];
  int32_t bf16[LLATTN_CAST_MAX_SEGS];
  int32_t vec[LLATTN_CAST_MAX_SEGS];  // source and destination 16-byte aligned: vector loads and stores
  int32_t nseg;
};

__global__ __launch_bounds__(256) void cast_kernel(const CastArgs a) {
  const int64_t total = a.start[a.nseg];
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < total; c += (int64_t)gridDim.x * 256) {
    int s = 0;
    while (s + 1 < a.nseg && c >= a.start[s + 1]) ++s;
    const int64_t e0 = (c - a.start[s]) * 8;  // first element of the chunk within segment s
    const float* src = a.src[s] + e0;
    const int64_t left = a.n[s] - e0;
    if (left >= 8 && a.vec[s]) {
      const float4 u = reinterpret_cast<const float4*>(src)[0], v = reinterpret_cast<const float4*>(src)[1];
      if (a.bf16[s]) {
        uint16_t* d = static_cast<uint16_t*>(a.dst[s]) + e0;
        *reinterpret_cast<uint4*>(d) = make_uint4(pack_bf16x2(u.x, u.y), pack_bf16x2(u.z, u.w),
                                                  pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
      } else {
        float4* d = reinterpret_cast<float4*>(static_cast<float*>(a.dst[s]) + e0);
        d[0] = u;
        d[1] = v;
      }
    } else {  // the segment's last, partial chunk, or a misaligned segment
      for (int64_t i = 0; i < min(left, (int64_t)8); ++i) {
        if (a.bf16[s]) static_cast<uint16_t*>(a.dst[s])[e0 + i] = f2bf(src[i]);
        else static_cast<float*>(a.dst[s])[e0 + i] = src[i];
      }
    }
  }
}

// dst[c][r] = src[r][c] for a bf16 matrix, in 64 x 64 tiles through LDS: 16-byte row reads of src and 16-byte
// row writes of dst (rows and columns multiples of 8).  The padded LDS rows (72 elements) spread the
// transposing element writes over the banks.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const uint16_t* __restrict__ src, int64_t lds, int rows,
                                                             int cols, uint16_t* __restrict__ dst, int64_t ldd) {
  __shared__ uint16_t t[64][72];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64, tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = tid + 256 * i, rl = q >> 3, cl = 8 * (q & 7);
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (r0 + rl < rows && c0 + cl < cols) v = *reinterpret_cast<const uint4*>(src + (int64_t)(r0 + rl) * lds + c0 + cl);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      t[cl + 2 * e][rl] = (uint16_t)(w[e] & 0xffffu);
      t[cl + 2 * e + 1][rl] = (uint16_t)(w[e] >> 16);
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = tid + 256 * i, cl = q >> 3, rl = 8 * (q & 7);
    if (c0 + cl < cols && r0 + rl < rows)
      *reinterpret_cast<uint4*>(dst + (int64_t)(c0 + cl) * ldd + r0 + rl) = *reinterpret_cast<const uint4*>(&t[cl][rl]);
  }
}

}  // namespace
}  // namespace llattn

using namespace llattn;

extern "C" int32_t llattn_transpose(const void* src, int64_t ld_src, int32_t rows, int32_t cols, void* dst,
                                    int64_t ld_dst, void* stream) {
  if (rows <= 0 || cols <= 0 || rows % 8 || cols % 8)
    return fail(LLATTN_ERR_SHAPE, "llattn_transpose: rows %d and cols %d must be positive multiples of 8", rows, cols);
  if (!src || !dst || !aligned16(src) || !aligned16(dst) || ld_src % 8 || ld_dst % 8 || ld_src < cols || ld_dst < rows)
    return fail(LLATTN_ERR_LAYOUT, "llattn_transpose: 16-byte aligned matrices with leading dimensions >= their rows, "
                "multiples of 8, needed");
  const dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
  hipLaunchKernelGGL(transpose_bf16_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(src), ld_src, rows, cols, static_cast<uint16_t*>(dst), ld_dst);
  return check_launch("llattn_transpose");
}

extern "C" int32_t llattn_cast(int32_t nseg, const float* const* src, void* const* dst, const int64_t* n,
                               const int32_t* dst_dtype, void* stream) {
  if (nseg < 1 || nseg > LLATTN_CAST_MAX_SEGS)
    return fail(LLATTN_ERR_SHAPE, "llattn_cast: %d segments (1 to %d supported)", nseg, LLATTN_CAST_MAX_SEGS);
  if (!src || !dst || !n || !dst_dtype) return fail(LLATTN_ERR_LAYOUT, "llattn_cast: null argument array");
  CastArgs a{};
  a.nseg = nseg;
  int64_t chunks = 0;
  for (int i = 0; i < nseg; ++i) {
    if (n[i] < 0) return fail(LLATTN_ERR_SHAPE, "llattn_cast: segment %d has negative length %lld", i, (long long)n[i]);
    if (dst_dtype[i] != LLATTN_BF16 && dst_dtype[i] != LLATTN_F32)
      return fail(LLATTN_ERR_DTYPE, "llattn_cast: segment %d has unknown output dtype %d", i, dst_dtype[i]);
    if (n[i] > 0 && (!src[i] || !dst[i] || (uintptr_t)src[i] % 4 || (uintptr_t)dst[i] % (dst_dtype[i] == LLATTN_BF16 ? 2 : 4)))
      return fail(LLATTN_ERR_LAYOUT, "llattn_cast: segment %d arrays must be non-null and element-aligned", i);
    a.src[i] = src[i];
    a.dst[i] = dst[i];
    a.n[i] = n[i];
    a.bf16[i] = dst_dtype[i] == LLATTN_BF16;
    a.vec[i] = aligned16(src[i]) && aligned16(dst[i]);
    a.start[i] = chunks;
    chunks += (n[i] + 7) / 8;
  }
  a.start[nseg] = chunks;
  if (chunks == 0) return LLATTN_OK;
  const int64_t blocks = std::min<int64_t>((chunks + 255) / 256, 4096);
  hipLaunchKernelGGL(cast_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("llattn_cast");
}
