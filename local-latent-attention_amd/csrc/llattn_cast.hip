// fp32 -> bf16 (or fp32 -> fp32) copies of several arrays in one launch: the weight casts that bf16
// autocast performs once per forward for every nn.Linear of the block, and the concatenated biases
// of projections that share one GEMM.  HBM-bound; one pass over each array.
//
// Plain segments: the launch covers their concatenation in chunks of 8 elements (32 bytes read); each
// thread finds its segment by a scan over the (at most LLATTN_CAST_MAX_SEGS) segment starts.  Segments whose
// source and destination are 16-byte aligned move with 16-byte loads and stores, others element by element.
// Segments that also want a transposed bf16 copy (the weights whose input gradients run as dy (W^T)^T) are
// cut into 64 x 64 tiles, one workgroup each, placed before the chunk workgroups: each tile is read once
// (fp32 rows), written as bf16 rows, and written again transposed through LDS, so W^T costs 2 bytes per
// element on top of the cast instead of a separate read and write of W.
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
  uint16_t* tdst[LLATTN_CAST_MAX_SEGS];  // non-null: segment written in tiles, transposed copy here
  int64_t tld[LLATTN_CAST_MAX_SEGS];     // leading dimension of tdst (elements)
  int32_t rows[LLATTN_CAST_MAX_SEGS];    // the tiled segment as a row-major [rows][n / rows] matrix
  int32_t tile_start[LLATTN_CAST_MAX_SEGS + 1];  // first tile workgroup of segment i (tiled segments only)
  int32_t nseg;
};

// One 64 x 64 tile of a tiled segment: fp32 rows in (16-byte loads), bf16 rows out (8-byte stores), and the
// transposed bf16 tile out through LDS (16-byte stores of 8 consecutive rows).  rows and cols are multiples
// of 8, so a 4-column load group and an 8-row store group are either wholly inside the matrix or wholly out.
__device__ __forceinline__ void cast_tile(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                          uint16_t* __restrict__ tdst, int64_t tld, int rows, int cols, int tile,
                                          uint16_t (*t)[72]) {
  const int tiles_c = (cols + 63) >> 6;
  const int r0 = (tile / tiles_c) * 64, c0 = (tile % tiles_c) * 64, tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = tid + 256 * i, rl = q >> 4, cl = 4 * (q & 15);
    float4 u = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r0 + rl < rows && c0 + cl < cols) {
      const int64_t e = (int64_t)(r0 + rl) * cols + c0 + cl;
      u = *reinterpret_cast<const float4*>(src + e);
      *reinterpret_cast<uint2*>(dst + e) = make_uint2(pack_bf16x2(u.x, u.y), pack_bf16x2(u.z, u.w));
    }
    t[cl][rl] = f2bf(u.x);
    t[cl + 1][rl] = f2bf(u.y);
    t[cl + 2][rl] = f2bf(u.z);
    t[cl + 3][rl] = f2bf(u.w);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = tid + 256 * i, cl = q >> 3, rl = 8 * (q & 7);
    if (c0 + cl < cols && r0 + rl < rows)
      *reinterpret_cast<uint4*>(tdst + (int64_t)(c0 + cl) * tld + r0 + rl) = *reinterpret_cast<const uint4*>(&t[cl][rl]);
  }
}

__global__ __launch_bounds__(256) void cast_kernel(const CastArgs a) {
  __shared__ uint16_t t[64][72];
  const int tiles = a.tile_start[a.nseg];
  if ((int)blockIdx.x < tiles) {  // a tile of a transposed segment (workgroup-uniform branch)
    int s = 0;
    while (s + 1 < a.nseg && (int)blockIdx.x >= a.tile_start[s + 1]) ++s;
    const int rows = a.rows[s];
    cast_tile(a.src[s], static_cast<uint16_t*>(a.dst[s]), a.tdst[s], a.tld[s], rows, (int)(a.n[s] / rows),
              (int)blockIdx.x - a.tile_start[s], t);
    return;
  }
  const int64_t total = a.start[a.nseg];
  const int64_t nblk = (int64_t)gridDim.x - tiles;
  for (int64_t c = ((int64_t)blockIdx.x - tiles) * 256 + threadIdx.x; c < total; c += nblk * 256) {
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

extern "C" int32_t llattn_cast_transposed(int32_t nseg, const float* const* src, void* const* dst,
                                          const int64_t* n, const int32_t* dst_dtype, void* const* dst_t,
                                          const int64_t* ld_t, const int32_t* rows, void* stream) {
  if (nseg < 1 || nseg > LLATTN_CAST_MAX_SEGS)
    return fail(LLATTN_ERR_SHAPE, "llattn_cast: %d segments (1 to %d supported)", nseg, LLATTN_CAST_MAX_SEGS);
  if (!src || !dst || !n || !dst_dtype) return fail(LLATTN_ERR_LAYOUT, "llattn_cast: null argument array");
  if (dst_t && (!ld_t || !rows))
    return fail(LLATTN_ERR_LAYOUT, "llattn_cast_transposed: dst_t given without ld_t and rows");
  CastArgs a{};
  a.nseg = nseg;
  int64_t chunks = 0, tiles = 0;
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
    a.tile_start[i] = (int32_t)tiles;
    if (dst_t && dst_t[i] && n[i] > 0) {
      const int64_t r = rows[i], c = r > 0 ? n[i] / r : 0;
      if (r <= 0 || r * c != n[i] || r % 8 || c % 8 || r > (1 << 20) || c > (1 << 20))
        return fail(LLATTN_ERR_SHAPE, "llattn_cast_transposed: segment %d: %lld elements are not a [rows, cols] "
                    "matrix with rows = %d and both multiples of 8 (at most 2^20)", i, (long long)n[i], rows[i]);
      if (!a.bf16[i] || !a.vec[i] || !aligned16(dst_t[i]) || ld_t[i] % 8 || ld_t[i] < r)
        return fail(LLATTN_ERR_LAYOUT, "llattn_cast_transposed: segment %d: bf16 output, 16-byte aligned arrays "
                    "and a transposed leading dimension >= rows, a multiple of 8, needed", i);
      a.tdst[i] = static_cast<uint16_t*>(dst_t[i]);
      a.tld[i] = ld_t[i];
      a.rows[i] = (int32_t)r;
      tiles += ((r + 63) / 64) * ((c + 63) / 64);
      if (tiles > (1 << 30)) return fail(LLATTN_ERR_SHAPE, "llattn_cast_transposed: too many tiles");
    } else {
      chunks += (n[i] + 7) / 8;
    }
  }
  a.start[nseg] = chunks;
  a.tile_start[nseg] = (int32_t)tiles;
  if (chunks == 0 && tiles == 0) return LLATTN_OK;
  const int64_t blocks = tiles + std::min<int64_t>((chunks + 255) / 256, 4096);
  hipLaunchKernelGGL(cast_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("llattn_cast");
}

extern "C" int32_t llattn_cast(int32_t nseg, const float* const* src, void* const* dst, const int64_t* n,
                               const int32_t* dst_dtype, void* stream) {
  return llattn_cast_transposed(nseg, src, dst, n, dst_dtype, nullptr, nullptr, nullptr, stream);
}
