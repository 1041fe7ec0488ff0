// Cross entropy of bf16 logit rows with its gradient in the same pass, for the LM head of the
// training step (reference train.py:354-370: F.cross_entropy over [B*T, V] bf16 logits, computed in
// fp32 under autocast, and logits.argmax(-1) for the accuracy metric).
//
// One 256-thread workgroup per row.  The row (V <= 65536 bf16, at most 128 KB) is read once into
// registers as 16-byte pieces (thread t holds pieces t, t + 256, ...); the row maximum and its first
// index, then the sum of exp(x - max), come from fixed-order reductions over the threads, so the
// result does not depend on timing.  With a gradient requested, every logit is replaced by
//   d = (softmax(x)_j - [j == target]) * scale
// rounded to bf16 (the in-place dlogits of a chunked head), written after every read of the row.
// HBM traffic per row: V * 2 bytes read, V * 2 bytes written (gradient), 8 bytes of results.
#include "llattn_abi.h"
#include "llattn_device.h"

namespace llattn {
namespace {

struct XentArgs {
  const uint16_t* logits;
  int64_t ld;
  uint16_t* dlogits;  // may equal logits; null: no gradient
  int64_t ld_d;
  const int64_t* targets;
  int64_t ignore_index;
  const float* scale;  // device scalar: the gradient of the loss sum per row (1 / valid rows for a mean)
  float* loss;         // [rows]: logsumexp - x[target], 0 for ignored rows, NaN for targets outside [0, V)
  int32_t* pred;       // [rows] or null: first index of the row maximum
  int V;
};

constexpr float kNegInfX = -__builtin_huge_valf();

// (value, index) maximum with the smaller index on ties
__device__ __forceinline__ void max_first(float& m, int& i, float m2, int i2) {
  if (m2 > m || (m2 == m && i2 < i)) {
    m = m2;
    i = i2;
  }
}

template <int CPT>
__global__ __launch_bounds__(256) void xent_kernel(const XentArgs a) {
  __shared__ float sm[4], ss[4], sxt;
  __shared__ int si[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const int nch = a.V >> 3;
  const uint16_t* src = a.logits + row * a.ld;
  const int64_t tgt = a.targets[row];
  const bool ignored = tgt == a.ignore_index;
  const bool bad = !ignored && (tgt < 0 || tgt >= a.V);

  uint4 u[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + 256 * i;
    u[i] = c < nch ? *reinterpret_cast<const uint4*>(src + 8 * c) : make_uint4(0u, 0u, 0u, 0u);
  }
  auto val = [&](int i, int e) {  // element e (0..7) of piece i as fp32
    const uint32_t w = e < 2 ? u[i].x : e < 4 ? u[i].y : e < 6 ? u[i].z : u[i].w;
    return (e & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
  };

  // row maximum and its first index; the thread holding the target keeps its logit
  float m = kNegInfX;
  int mi = 0x7fffffff;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + 256 * i;
    if (c < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) max_first(m, mi, val(i, e), 8 * c + e);
      if (!ignored && !bad && (tgt >> 3) == c) sxt = val(i, (int)(tgt & 7));
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) max_first(m, mi, __shfl_xor(m, o), __shfl_xor(mi, o));
  if (lane == 0) {
    sm[wave] = m;
    si[wave] = mi;
  }
  __syncthreads();
  m = sm[0];
  mi = si[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) max_first(m, mi, sm[w], si[w]);

  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    if (tid + 256 * i < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s += __expf(val(i, e) - m);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if (lane == 0) ss[wave] = s;
  __syncthreads();  // every read of the row is done: the gradient may overwrite it
  s = (ss[0] + ss[1]) + (ss[2] + ss[3]);
  const float lse = m + __logf(s);

  if (tid == 0) {
    a.loss[row] = ignored ? 0.f : bad ? __builtin_nanf("") : lse - sxt;
    if (a.pred) a.pred[row] = mi;
  }
  if (a.dlogits) {
    const float sc = ignored ? 0.f : *a.scale;
    uint16_t* dst = a.dlogits + row * a.ld_d;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + 256 * i;
      if (c >= nch) continue;
      float g[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float p = __expf(val(i, e) - lse);
        g[e] = (8 * c + e == tgt ? p - 1.f : p) * sc;
      }
      *reinterpret_cast<uint4*>(dst + 8 * c) =
          make_uint4(pack_bf16x2(g[0], g[1]), pack_bf16x2(g[2], g[3]), pack_bf16x2(g[4], g[5]), pack_bf16x2(g[6], g[7]));
    }
  }
}

}  // namespace
}  // namespace llattn

using namespace llattn;

extern "C" int32_t llattn_xent(const void* logits, int64_t ld, int32_t rows, int32_t V, const int64_t* targets,
                               int64_t ignore_index, float* loss, int32_t* pred, void* dlogits, int64_t ld_d,
                               const float* grad_scale, void* stream) {
  if (rows < 0 || V < 8 || V % 8 || V > 256 * 8 * 32)
    return fail(LLATTN_ERR_SHAPE, "llattn_xent: rows %d, V %d (V a multiple of 8 in [8, 65536])", rows, V);
  if (rows == 0) return LLATTN_OK;
  if (!logits || !targets || !loss) return fail(LLATTN_ERR_LAYOUT, "llattn_xent: null logits, targets or loss");
  if (ld < V || ld % 8 || !aligned16(logits))
    return fail(LLATTN_ERR_LAYOUT, "llattn_xent: logits need 16-byte aligned rows (ld %lld >= V, multiple of 8)",
                (long long)ld);
  if (dlogits && (ld_d < V || ld_d % 8 || !aligned16(dlogits) || !grad_scale))
    return fail(LLATTN_ERR_LAYOUT, "llattn_xent: dlogits need 16-byte aligned rows (ld_d %lld) and a grad_scale",
                (long long)ld_d);
  if (dlogits && dlogits != logits) {  // distinct buffers must not overlap
    const char* l0 = static_cast<const char*>(logits);
    const char* d0 = static_cast<const char*>(dlogits);
    const int64_t lb = ((int64_t)(rows - 1) * ld + V) * 2, db = ((int64_t)(rows - 1) * ld_d + V) * 2;
    if (d0 < l0 + lb && l0 < d0 + db)
      return fail(LLATTN_ERR_LAYOUT, "llattn_xent: dlogits overlaps logits without being the same buffer");
  }
  XentArgs a{static_cast<const uint16_t*>(logits), ld, static_cast<uint16_t*>(dlogits), ld_d, targets,
             ignore_index, grad_scale, loss, pred, V};
  const int nch = V / 8;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)rows), block(256);
  if (nch <= 256 * 4) hipLaunchKernelGGL(xent_kernel<4>, grid, block, 0, st, a);
  else if (nch <= 256 * 8) hipLaunchKernelGGL(xent_kernel<8>, grid, block, 0, st, a);
  else if (nch <= 256 * 16) hipLaunchKernelGGL(xent_kernel<16>, grid, block, 0, st, a);
  else hipLaunchKernelGGL(xent_kernel<32>, grid, block, 0, st, a);
  return check_launch("llattn_xent");
}
