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

}  // namespace
}  // namespace llattn

using namespace llattn;

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
