// Chunk-causal latent attention, forward and backward, for gfx950.
//
// Semantics (reference models.py:361-375): latent query s of head lh attends
// latents n < c(s), where c(s) = (s * q_block) / chunk is the chunk id of the
// query's first token (token-wise queries: q_block = 1); scale 1/sqrt(Ldh);
// queries with c(s) = 0 output 0.
//
// One thread owns one latent query (its Ldh-vector lives in registers); a
// 256-thread workgroup covers 256 queries of one (batch, latent head) and
// streams the latent keys/values it can see through LDS.  The latent count is
// small (16 at the 0.55b shape, 256 at the long-context shape), so the work is
// a bandwidth-bound pass over the queries.  The backward reduces the dgk / dgv
// contributions of a wave with a halving butterfly (each step exchanges half of
// the remaining vector), combines the four waves in LDS, writes one partial per
// workgroup and sums the partials in tile order in a second kernel: no atomics,
// bitwise deterministic.
#include "llattn_abi.h"
#include "llattn_device.h"

namespace llattn {

struct LatentArgs {
  int B, Lh, Ldh, n_q, q_block, chunk, n_chunks, n_tiles;
  float scale, scale_log2;
  const void* rq; int64_t rq_sb, rq_sn, rq_sh;
  const void* gk; int64_t gk_sb, gk_sn, gk_sh;
  const void* gv; int64_t gv_sb, gv_sn, gv_sh;
  const void* out; int64_t o_sb, o_sn, o_sh;
  float* lse;  // [B][Lh][n_q]
  const void* dout; int64_t do_sb, do_sn, do_sh;
  void* drq; int64_t drq_sb, drq_sn, drq_sh;
  void* dgk; int64_t dgk_sb, dgk_sn, dgk_sh;
  void* dgv; int64_t dgv_sb, dgv_sn, dgv_sh;
  float* part;  // [B*Lh*n_tiles][n_chunks][2][Ldh]
};

constexpr int kQTile = 256;

// number of latents visible to latent query s
__device__ __forceinline__ int visible(int s, const LatentArgs& a) {
  return min((int)(((int64_t)s * a.q_block) / a.chunk), a.n_chunks);
}

template <typename T, int LDP>
__device__ __forceinline__ void load_vec(float (&v)[LDP], const T* p, int Ldh, bool valid) {
#pragma unroll
  for (int d = 0; d < LDP; d += 4) {
    if (valid && d < Ldh) {
      load4<T>(p + d, &v[d]);
    } else {
      v[d] = v[d + 1] = v[d + 2] = v[d + 3] = 0.f;
    }
  }
}

// latents [n0, n0+NL) of one (b, lh) into LDS as fp32 rows (zero past n_end / Ldh)
template <typename T, int LDP, int NL>
__device__ __forceinline__ void stage_latents(float (*gks)[LDP], float (*gvs)[LDP], const T* gk, int64_t gk_sn,
                                              const T* gv, int64_t gv_sn, int n0, int n_end, int Ldh) {
  for (int idx = threadIdx.x; idx < NL * (LDP / 4); idx += 256) {
    const int n = idx / (LDP / 4), d = (idx % (LDP / 4)) * 4, nn = n0 + n;
    float kv[4] = {0.f, 0.f, 0.f, 0.f}, vv[4] = {0.f, 0.f, 0.f, 0.f};
    if (nn < n_end && d < Ldh) {
      load4<T>(gk + (int64_t)nn * gk_sn + d, kv);
      load4<T>(gv + (int64_t)nn * gv_sn + d, vv);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      gks[n][d + j] = kv[j];
      gvs[n][d + j] = vv[j];
    }
  }
}

template <typename T, int LDP>
__global__ __launch_bounds__(256) void latent_fwd_kernel(const LatentArgs a) {
  constexpr int NL = 64;
  __shared__ __align__(16) float gks[NL][LDP];
  __shared__ __align__(16) float gvs[NL][LDP];
  const int tile = blockIdx.x % a.n_tiles, bh = blockIdx.x / a.n_tiles, lh = bh % a.Lh, b = bh / a.Lh;
  const int s = tile * kQTile + threadIdx.x;
  const bool sv = s < a.n_q;
  const int ncq = sv ? visible(s, a) : 0;
  const int nmax = visible(min(tile * kQTile + kQTile - 1, a.n_q - 1), a);

  const T* gkb = static_cast<const T*>(a.gk) + b * a.gk_sb + lh * a.gk_sh;
  const T* gvb = static_cast<const T*>(a.gv) + b * a.gv_sb + lh * a.gv_sh;
  float q[LDP], acc[LDP];
  load_vec<T, LDP>(q, static_cast<const T*>(a.rq) + b * a.rq_sb + lh * a.rq_sh + (int64_t)s * a.rq_sn, a.Ldh, sv);
#pragma unroll
  for (int d = 0; d < LDP; ++d) acc[d] = 0.f;
  float m = kNegInf, l = 0.f;
  for (int n0 = 0; n0 < nmax; n0 += NL) {
    __syncthreads();
    stage_latents<T, LDP, NL>(gks, gvs, gkb, a.gk_sn, gvb, a.gv_sn, n0, nmax, a.Ldh);
    __syncthreads();
    const int nend = min(NL, ncq - n0);
    for (int n = 0; n < nend; ++n) {
      float sc = 0.f;
#pragma unroll
      for (int d = 0; d < LDP; ++d) sc += q[d] * gks[n][d];
      sc *= a.scale_log2;
      const float m_new = fmaxf(m, sc);
      const float alpha = fast_exp2(m - m_new);
      const float p = fast_exp2(sc - m_new);
      l = l * alpha + p;
#pragma unroll
      for (int d = 0; d < LDP; ++d) acc[d] = acc[d] * alpha + p * gvs[n][d];
      m = m_new;
    }
  }
  if (sv) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    T* op = static_cast<T*>(const_cast<void*>(a.out)) + b * a.o_sb + lh * a.o_sh + (int64_t)s * a.o_sn;
#pragma unroll
    for (int d = 0; d < LDP; d += 4) {
      if (d < a.Ldh) {
        float v4[4] = {acc[d] * inv, acc[d + 1] * inv, acc[d + 2] * inv, acc[d + 3] * inv};
        store4<T>(op + d, v4);
      }
    }
    a.lse[((int64_t)b * a.Lh + lh) * a.n_q + s] = l > 0.f ? (m + __log2f(l)) * kLn2 : kNegInf;
  }
}

// Halving butterfly: on entry every lane holds a length-M vector; on exit lane
// `lane` holds element (lane >> (6 - log2 M)) of the wave-wide sum (M <= 64).
template <int M, int O>
__device__ __forceinline__ void butterfly(float* v, int lane) {
  if constexpr (O > 0) {
    if constexpr (M > 1) {
      constexpr int H = M / 2;
      const bool up = (lane & O) != 0;
#pragma unroll
      for (int j = 0; j < H; ++j) {
        const float keep = up ? v[j + H] : v[j];
        const float send = up ? v[j] : v[j + H];
        v[j] = keep + __shfl_xor(send, O);
      }
      butterfly<H, O / 2>(v, lane);
    } else {
      v[0] += __shfl_xor(v[0], O);
      butterfly<1, O / 2>(v, lane);
    }
  }
}
template <int M>
constexpr int log2i() { return M <= 1 ? 0 : 1 + log2i<M / 2>(); }

template <typename T, int LDP>
__global__ __launch_bounds__(256) void latent_bwd_kernel(const LatentArgs a) {
  constexpr int NL = 16, SHIFT = 6 - log2i<LDP>();
  __shared__ __align__(16) float gks[NL][LDP];
  __shared__ __align__(16) float gvs[NL][LDP];
  __shared__ float red[4][NL][2][LDP];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tile = blockIdx.x % a.n_tiles, bh = blockIdx.x / a.n_tiles, lh = bh % a.Lh, b = bh / a.Lh;
  const int s = tile * kQTile + threadIdx.x;
  const bool sv = s < a.n_q;
  const int ncq = sv ? visible(s, a) : 0;
  const int nmax = visible(min(tile * kQTile + kQTile - 1, a.n_q - 1), a);

  const T* gkb = static_cast<const T*>(a.gk) + b * a.gk_sb + lh * a.gk_sh;
  const T* gvb = static_cast<const T*>(a.gv) + b * a.gv_sb + lh * a.gv_sh;
  float q[LDP], dl[LDP], drq[LDP], c[LDP];
  load_vec<T, LDP>(q, static_cast<const T*>(a.rq) + b * a.rq_sb + lh * a.rq_sh + (int64_t)s * a.rq_sn, a.Ldh, sv);
  load_vec<T, LDP>(dl, static_cast<const T*>(a.dout) + b * a.do_sb + lh * a.do_sh + (int64_t)s * a.do_sn, a.Ldh, sv);
#pragma unroll
  for (int d = 0; d < LDP; ++d) drq[d] = 0.f;
  const float lse_nat = sv ? a.lse[((int64_t)b * a.Lh + lh) * a.n_q + s] : kNegInf;
  const float lse2 = lse_nat == kNegInf ? 0.f : lse_nat * kLog2e;

  // pass 1: D = sum_n P_n (dL . gv_n) in fp32 from the recomputed weights.  (dL . L with L read back
  // at storage precision would cancel badly when the latent softmax is peaked.)
  float Dsum = 0.f;
  for (int n0 = 0; n0 < nmax; n0 += NL) {
    __syncthreads();
    stage_latents<T, LDP, NL>(gks, gvs, gkb, a.gk_sn, gvb, a.gv_sn, n0, nmax, a.Ldh);
    __syncthreads();
    const int nend = min(NL, ncq - n0);
    for (int n = 0; n < nend; ++n) {
      float sc = 0.f, dp = 0.f;
#pragma unroll
      for (int d = 0; d < LDP; ++d) {
        sc += q[d] * gks[n][d];
        dp += dl[d] * gvs[n][d];
      }
      Dsum += fast_exp2(sc * a.scale_log2 - lse2) * dp;
    }
  }
  float* part = a.part + (((int64_t)b * a.Lh + lh) * a.n_tiles + tile) * a.n_chunks * 2 * a.Ldh;

  // pass 2: dS, drq and the per-workgroup dgk / dgv partials
  for (int n0 = 0; n0 < nmax; n0 += NL) {
    __syncthreads();
    stage_latents<T, LDP, NL>(gks, gvs, gkb, a.gk_sn, gvb, a.gv_sn, n0, nmax, a.Ldh);
    __syncthreads();
    const int cnt = min(NL, nmax - n0);  // uniform over the workgroup
    for (int n = 0; n < cnt; ++n) {
      float sc = 0.f, dp = 0.f;
#pragma unroll
      for (int d = 0; d < LDP; ++d) {
        sc += q[d] * gks[n][d];
        dp += dl[d] * gvs[n][d];
      }
      const float p = (n0 + n < ncq) ? fast_exp2(sc * a.scale_log2 - lse2) : 0.f;
      const float ds = p * (dp - Dsum) * a.scale;
#pragma unroll
      for (int d = 0; d < LDP; ++d) {
        drq[d] += ds * gks[n][d];
        c[d] = ds * q[d];
      }
      butterfly<LDP, 32>(c, lane);
      if ((lane & ((1 << SHIFT) - 1)) == 0) red[wave][n][0][lane >> SHIFT] = c[0];
#pragma unroll
      for (int d = 0; d < LDP; ++d) c[d] = p * dl[d];
      butterfly<LDP, 32>(c, lane);
      if ((lane & ((1 << SHIFT) - 1)) == 0) red[wave][n][1][lane >> SHIFT] = c[0];
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < cnt * 2 * a.Ldh; idx += 256) {
      const int n = idx / (2 * a.Ldh), rem = idx % (2 * a.Ldh), which = rem / a.Ldh, d = rem % a.Ldh;
      part[(int64_t)(n0 + n) * 2 * a.Ldh + which * a.Ldh + d] =
          red[0][n][which][d] + red[1][n][which][d] + red[2][n][which][d] + red[3][n][which][d];
    }
  }
  if (sv) {
    T* p = static_cast<T*>(a.drq) + b * a.drq_sb + lh * a.drq_sh + (int64_t)s * a.drq_sn;
#pragma unroll
    for (int d = 0; d < LDP; d += 4)
      if (d < a.Ldh) store4<T>(p + d, &drq[d]);
  }
}

// dgk / dgv [b][n][lh][d] = sum over query tiles (in tile order) of the partials;
// tiles whose queries see fewer than n+1 latents wrote nothing for n.
template <typename T>
__global__ __launch_bounds__(256) void latent_reduce_kernel(const LatentArgs a) {
  const int64_t total = (int64_t)a.B * a.Lh * a.n_chunks * 2 * a.Ldh;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    int64_t rest = idx;
    const int d = rest % a.Ldh; rest /= a.Ldh;
    const int which = rest % 2; rest /= 2;
    const int n = rest % a.n_chunks; rest /= a.n_chunks;
    const int lh = rest % a.Lh;
    const int b = rest / a.Lh;
    const float* p = a.part + ((int64_t)b * a.Lh + lh) * a.n_tiles * a.n_chunks * 2 * a.Ldh +
                     (int64_t)n * 2 * a.Ldh + which * a.Ldh + d;
    float s = 0.f;
    for (int t = 0; t < a.n_tiles; ++t) {
      if (visible(min(t * kQTile + kQTile - 1, a.n_q - 1), a) > n) s += p[(int64_t)t * a.n_chunks * 2 * a.Ldh];
    }
    T* out = which == 0 ? static_cast<T*>(a.dgk) + b * a.dgk_sb + lh * a.dgk_sh + (int64_t)n * a.dgk_sn + d
                        : static_cast<T*>(a.dgv) + b * a.dgv_sb + lh * a.dgv_sh + (int64_t)n * a.dgv_sn + d;
    *out = from_f<T>(s);
  }
}

namespace {

template <typename T, int LDP>
void launch(bool fwd, const LatentArgs& a, hipStream_t st) {
  const dim3 grid(a.B * a.Lh * a.n_tiles);
  if (fwd) {
    hipLaunchKernelGGL((latent_fwd_kernel<T, LDP>), grid, dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL((latent_bwd_kernel<T, LDP>), grid, dim3(256), 0, st, a);
    const int64_t total = (int64_t)a.B * a.Lh * a.n_chunks * 2 * a.Ldh;
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
    hipLaunchKernelGGL((latent_reduce_kernel<T>), dim3(blocks), dim3(256), 0, st, a);
  }
}
template <typename T>
bool dispatch(int ldp, bool fwd, const LatentArgs& a, hipStream_t st) {
  switch (ldp) {
    case 8: launch<T, 8>(fwd, a, st); return true;
    case 16: launch<T, 16>(fwd, a, st); return true;
    case 32: launch<T, 32>(fwd, a, st); return true;
    case 64: launch<T, 64>(fwd, a, st); return true;
    default: return false;
  }
}

int32_t common(const llattn_shape* s, const llattn_tensor* rq, const llattn_tensor* gk, const llattn_tensor* gv,
               LatentArgs* a) {
  int32_t rc = check_shape(s);
  if (rc) return rc;
  if ((rc = check_view("rq", rq, s->dtype, true)) || (rc = check_view("gk", gk, s->dtype, true)) ||
      (rc = check_view("gv", gv, s->dtype, true)))
    return rc;
  *a = LatentArgs{};
  a->B = s->B; a->Lh = s->Lh; a->Ldh = s->Ldh; a->n_q = s->n_q; a->q_block = s->q_block;
  a->chunk = s->chunk; a->n_chunks = s->n_chunks; a->n_tiles = (s->n_q + kQTile - 1) / kQTile;
  a->scale = 1.0f / sqrtf((float)s->Ldh);
  a->scale_log2 = a->scale * kLog2e;
  a->rq = rq->ptr; a->rq_sb = rq->sb; a->rq_sn = rq->sn; a->rq_sh = rq->sh;
  a->gk = gk->ptr; a->gk_sb = gk->sb; a->gk_sn = gk->sn; a->gk_sh = gk->sh;
  a->gv = gv->ptr; a->gv_sb = gv->sb; a->gv_sn = gv->sn; a->gv_sh = gv->sh;
  return LLATTN_OK;
}

}  // namespace
}  // namespace llattn

using namespace llattn;

extern "C" int32_t llattn_latent_fwd(const llattn_shape* s, const llattn_tensor* rq, const llattn_tensor* gk,
                                     const llattn_tensor* gv, const llattn_tensor* out, float* lse, void* stream) {
  LatentArgs a;
  int32_t rc = common(s, rq, gk, gv, &a);
  if (rc) return rc;
  if ((rc = check_view("latent_out", out, s->dtype, true))) return rc;
  if (!lse) return fail(LLATTN_ERR_LAYOUT, "lse output must be non-null");
  a.out = out->ptr; a.o_sb = out->sb; a.o_sn = out->sn; a.o_sh = out->sh;
  a.lse = lse;
  const int ldp = padded_latent_dim(s->Ldh);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool ok = s->dtype == LLATTN_F32 ? dispatch<float>(ldp, true, a, st) : dispatch<uint16_t>(ldp, true, a, st);
  if (!ok) return fail(LLATTN_ERR_UNSUPPORTED, "latent head_dim %d unsupported", s->Ldh);
  return check_launch("llattn_latent_fwd");
}

extern "C" int32_t llattn_latent_bwd(const llattn_shape* s, const llattn_tensor* rq, const llattn_tensor* gk,
                                     const llattn_tensor* gv, const float* lse, const llattn_tensor* dout,
                                     const llattn_tensor* drq, const llattn_tensor* dgk, const llattn_tensor* dgv,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  LatentArgs a;
  int32_t rc = common(s, rq, gk, gv, &a);
  if (rc) return rc;
  if ((rc = check_view("dout", dout, s->dtype, true)) || (rc = check_view("drq", drq, s->dtype, true)) ||
      (rc = check_view("dgk", dgk, s->dtype, true)) || (rc = check_view("dgv", dgv, s->dtype, true)))
    return rc;
  if (!lse) return fail(LLATTN_ERR_LAYOUT, "lse must be non-null");
  const size_t need = llattn_workspace_size(s, LLATTN_WS_LATENT_BWD);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return fail(LLATTN_ERR_WORKSPACE, "latent backward needs %zu workspace bytes (got %zu)", need, workspace_bytes);
  a.lse = const_cast<float*>(lse);
  a.dout = dout->ptr; a.do_sb = dout->sb; a.do_sn = dout->sn; a.do_sh = dout->sh;
  a.drq = drq->ptr; a.drq_sb = drq->sb; a.drq_sn = drq->sn; a.drq_sh = drq->sh;
  a.dgk = dgk->ptr; a.dgk_sb = dgk->sb; a.dgk_sn = dgk->sn; a.dgk_sh = dgk->sh;
  a.dgv = dgv->ptr; a.dgv_sb = dgv->sb; a.dgv_sn = dgv->sn; a.dgv_sh = dgv->sh;
  a.part = static_cast<float*>(workspace);
  const int ldp = padded_latent_dim(s->Ldh);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool ok = s->dtype == LLATTN_F32 ? dispatch<float>(ldp, false, a, st) : dispatch<uint16_t>(ldp, false, a, st);
  if (!ok) return fail(LLATTN_ERR_UNSUPPORTED, "latent head_dim %d unsupported", s->Ldh);
  return check_launch("llattn_latent_bwd");
}
