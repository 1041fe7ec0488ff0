// Chunk-causal latent attention, forward and backward, for gfx950 (bf16/fp32 MFMA).
//
// Semantics (reference models.py:361-375): latent query s of latent head lh
// attends latents n < c(s), where c(s) = (s * q_block) / chunk is the chunk id
// of the query's first token (token-wise queries: q_block = 1), with scale
// 1/sqrt(Ldh); queries with c(s) = 0 output 0.
//
// The latents play the role of keys/values of a small attention, so the
// kernels reuse the tile machinery of the local kernels: one 256-thread
// workgroup per (batch, latent head, 64 queries), waves of 16 queries, latent
// tiles of 64 staged in LDS, S^T = GK RQ^T and O^T = GV^T P^T on MFMA.
//
// Backward, without atomics:
//   pass Q  (per query tile): D_s = sum_n P_sn (dL_s . gv_n) in fp32 from the
//           recomputed weights, then drq = scale * sum_n dS_sn gk_n;
//   pass KV (per 16-latent tile and query segment): dgk, dgv partial sums over
//           the segment's queries (the four waves split the query sub-tiles and
//           are summed in LDS in wave order); a last kernel adds the segment
//           partials in segment order.
//   With one latent tile (bf16, at most 16 latents) both passes run as one kernel
//   per query segment (latent_bwd_fused_kernel), with the products of the two.
#include "llattn_abi.h"
#include "llattn_device.h"

namespace llattn {

struct LatentArgs {
  int B, Lh, Ldh, n_q, q_block, chunk, n_chunks, n_qt, n_lt, n_seg, seg;  // seg: queries per segment
  float scale, scale_log2;
  const void* rq; int64_t rq_sb, rq_sn, rq_sh;
  const void* gk; int64_t gk_sb, gk_sn, gk_sh;
  const void* gv; int64_t gv_sb, gv_sn, gv_sh;
  void* out; int64_t o_sb, o_sn, o_sh;
  float* lse;  // [B][Lh][n_q]
  const void* dout; int64_t do_sb, do_sn, do_sh;
  void* drq; int64_t drq_sb, drq_sn, drq_sh;
  void* dgk; int64_t dgk_sb, dgk_sn, dgk_sh;
  void* dgv; int64_t dgv_sb, dgv_sn, dgv_sh;
  float* Dsum;  // workspace [B][Lh][n_q]
  float* part;  // workspace [B][Lh][n_seg][n_lt*16][2][Ldh]
};

// The one-pass backward (bf16, one latent tile of at most 16 latents, padded head dims up to 128)
bool latent_one_pass(int n_lt, bool bf16, int dhp) { return bf16 && n_lt == 1 && dhp <= 128; }

// Queries per segment of the latent-stationary pass (a multiple of 64): about 1024 workgroups (B Lh n_lt
// segments) fill the chip; segments stay at least 256 queries long, since each one adds fp32 partials
// (16 n_lt x 2 Ldh per (b, lh)) that are written and then read back by the ordered reduction.  The
// one-pass kernel (two workgroups per CU by its LDS) targets 512: one round of longer, pipelined segments
// (config 2: 49 us against 51 at 1024 and 256 workgroups).
int latent_seg(int B, int Lh, int n_chunks, int n_q, bool fused) {
  const int64_t units = (int64_t)B * Lh * ((n_chunks + 15) / 16);
  const int64_t wgs = fused ? 512 : 1024;
  const int64_t want = std::max<int64_t>(1, (wgs + units - 1) / units);  // segments per (b, lh, latent tile)
  const int64_t seg = ((n_q + want - 1) / want + 63) / 64 * 64;
  return (int)std::max<int64_t>(256, seg);
}

// number of latents visible to latent query s
__device__ __forceinline__ int visible(int s, const LatentArgs& a) {
  return min((int)(((int64_t)s * a.q_block) / a.chunk), a.n_chunks);
}

// ----------------------------------------------------------------------------
// forward
// ----------------------------------------------------------------------------
template <typename T, int DHP>
__global__ __launch_bounds__(256, DHP <= 64 ? 5 : 1) void latent_fwd_kernel(const LatentArgs a) {
  constexpr int DQ = DHP / 4, NT = DHP / 16, KP = DHP + kRowPad<T>;
  __shared__ __align__(16) T Ks[64 * KP];
  __shared__ __align__(16) T Vt[DHP * kTP];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane & 15, g = lane >> 4;
  const int qt = blockIdx.x % a.n_qt, bh = blockIdx.x / a.n_qt, lh = bh % a.Lh, b = bh / a.Lh;
  const int q0 = qt * 64, qw = q0 + 16 * wave, qi = qw + r;
  const bool qv = qi < a.n_q;
  const int ncq = qv ? visible(qi, a) : 0;
  const int nmax = visible(min(q0 + 63, a.n_q - 1), a);
  const int wmax = qw < a.n_q ? visible(min(qw + 15, a.n_q - 1), a) : 0;
  const T* gkb = static_cast<const T*>(a.gk) + b * a.gk_sb + lh * a.gk_sh;
  const T* gvb = static_cast<const T*>(a.gv) + b * a.gv_sb + lh * a.gv_sh;

  RowFrag<T, DQ> qf;
  qf.load(static_cast<const T*>(a.rq) + b * a.rq_sb + lh * a.rq_sh + (int64_t)qi * a.rq_sn, g, a.Ldh, qv);
  float m_run = kNegInf, l_run = 0.f;
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int n0 = 0; n0 < nmax; n0 += 64) {
    RowTile<T, DHP> tk;  // both tiles' loads in flight before the first LDS store waits for them
    TransTile<T, DHP> tv;
    tk.load(gkb, a.gk_sn, n0, nmax, a.Ldh);
    tv.load(gvb, a.gv_sn, n0, nmax, a.Ldh);
    lds_barrier();
    tk.template store<KP>(Ks);
    tv.store_t(Vt);
    lds_barrier();
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int s0 = n0 + 16 * st;
      if (s0 >= wmax) continue;  // uniform over the wave
      RowFrag<T, DQ> kf;
      kf.load_lds(Ks + (16 * st + r) * KP, g);
      const f32x4 s = row_mma(kf, qf, f32x4{0.f, 0.f, 0.f, 0.f});
      bool ok[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) ok[i] = s0 + 4 * g + i < ncq;
      online_softmax_pv<NT>(s, ok, a.scale_log2, m_run, l_run, acc, Vt + r * kTP + 16 * st + 4 * g);
    }
  }
  const float l = sum_groups(l_run);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (qv && g == 0 && a.lse)
    a.lse[((int64_t)b * a.Lh + lh) * a.n_q + qi] = l > 0.f ? (m_run + __log2f(l)) * kLn2 : kNegInf;
  if constexpr (std::is_same_v<T, uint16_t>) {
    // bf16: the wave's 16 output rows through its own LDS rows of Ks (after a barrier: every wave has read
    // its last key fragments), then 16-byte chunks in row order, so a store writes whole rows
    lds_barrier();
    T* sw = Ks + 16 * wave * KP;
#pragma unroll
    for (int t = 0; t < NT; ++t)
      *reinterpret_cast<uint2*>(sw + r * KP + 16 * t + 4 * g) =
          make_uint2(pack_bf16x2(acc[t][0] * inv, acc[t][1] * inv), pack_bf16x2(acc[t][2] * inv, acc[t][3] * inv));
    constexpr int CPR = DHP / 8;  // 16-byte chunks per row; 16 CPR is a multiple of 64
    static_assert((16 * CPR) % 64 == 0, "whole store instructions");
    T* obase = static_cast<T*>(a.out) + b * a.o_sb + lh * a.o_sh;
#pragma unroll
    for (int it = 0; it < 16 * CPR / 64; ++it) {
      const int idx = 64 * it + lane, rr = idx / CPR, c = idx % CPR, q = qw + rr;
      const uint4 x = *reinterpret_cast<const uint4*>(sw + rr * KP + 8 * c);
      if (q < a.n_q && 8 * c < a.Ldh) *reinterpret_cast<uint4*>(obase + (int64_t)q * a.o_sn + 8 * c) = x;
    }
  } else if (qv) {
    T* op = static_cast<T*>(a.out) + b * a.o_sb + lh * a.o_sh + (int64_t)qi * a.o_sn;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int d = 16 * t + 4 * g;
      if (d < a.Ldh) {
        float v4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v4[i] = acc[t][i] * inv;
        store4<T>(op + d, v4);
      }
    }
  }
}

// ----------------------------------------------------------------------------
// backward pass Q: D and drq
// ----------------------------------------------------------------------------
template <typename T, int DHP>
__global__ __launch_bounds__(256) void latent_bwd_q_kernel(const LatentArgs a) {
  constexpr int DQ = DHP / 4, NT = DHP / 16, KP = DHP + kRowPad<T>;
  __shared__ __align__(16) T Ks[64 * KP];
  __shared__ __align__(16) T Kt[DHP * kTP];
  __shared__ __align__(16) T Vs[64 * KP];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane & 15, g = lane >> 4;
  const int qt = blockIdx.x % a.n_qt, bh = blockIdx.x / a.n_qt, lh = bh % a.Lh, b = bh / a.Lh;
  const int q0 = qt * 64, qw = q0 + 16 * wave, qi = qw + r;
  const bool qv = qi < a.n_q;
  const int ncq = qv ? visible(qi, a) : 0;
  const int nmax = visible(min(q0 + 63, a.n_q - 1), a);
  const int wmax = qw < a.n_q ? visible(min(qw + 15, a.n_q - 1), a) : 0;
  const T* gkb = static_cast<const T*>(a.gk) + b * a.gk_sb + lh * a.gk_sh;
  const T* gvb = static_cast<const T*>(a.gv) + b * a.gv_sb + lh * a.gv_sh;
  const int64_t row = ((int64_t)b * a.Lh + lh) * a.n_q + qi;

  RowFrag<T, DQ> qf, dof;
  qf.load(static_cast<const T*>(a.rq) + b * a.rq_sb + lh * a.rq_sh + (int64_t)qi * a.rq_sn, g, a.Ldh, qv);
  dof.load(static_cast<const T*>(a.dout) + b * a.do_sb + lh * a.do_sh + (int64_t)qi * a.do_sn, g, a.Ldh, qv);
  // lse of a valid row, transformed only after the first latent tile is staged: a use right here would wait
  // for the query rows' loads before the tile's loads are even issued
  const float lse_raw = a.lse[((int64_t)b * a.Lh + lh) * a.n_q + min(qi, a.n_q - 1)];
  const bool single = nmax <= 64;  // one latent tile: stage it once for both passes

  // pass 1: D = sum_n P_n dP_n
  float D = 0.f;
  // keys (rows, and transposed when one tile serves both passes) and values, loads in flight together
  auto stage = [&](int n0, bool trans) {
    TransTile<T, DHP> tk;
    RowTile<T, DHP> tv;
    tk.load(gkb, a.gk_sn, n0, nmax, a.Ldh);
    tv.load(gvb, a.gv_sn, n0, nmax, a.Ldh);
    lds_barrier();
    tk.template store_rows<KP>(Ks);
    if (trans) tk.store_t(Kt);
    tv.template store<KP>(Vs);
    lds_barrier();
  };
  if (nmax > 0) stage(0, single);
  const float lse2 = (!qv || lse_raw == kNegInf) ? 0.f : lse_raw * kLog2e;
  for (int n0 = 0; n0 < nmax; n0 += 64) {
    if (n0 > 0) stage(n0, single);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int s0 = n0 + 16 * st;
      if (s0 >= wmax) continue;
      RowFrag<T, DQ> kf, vf;
      kf.load_lds(Ks + (16 * st + r) * KP, g);
      vf.load_lds(Vs + (16 * st + r) * KP, g);
      const f32x4 s = row_mma(kf, qf, f32x4{0.f, 0.f, 0.f, 0.f});
      const f32x4 dp = row_mma(vf, dof, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (s0 + 4 * g + i < ncq) D += fast_exp2(s[i] * a.scale_log2 - lse2) * dp[i];
    }
  }
  D = sum_groups(D);
  if (qv && g == 0) a.Dsum[row] = D;

  // pass 2: drq^T += GK^T dS^T
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int n0 = 0; n0 < nmax; n0 += 64) {
    if (!single) stage(n0, true);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int s0 = n0 + 16 * st;
      if (s0 >= wmax) continue;
      RowFrag<T, DQ> kf, vf;
      kf.load_lds(Ks + (16 * st + r) * KP, g);
      vf.load_lds(Vs + (16 * st + r) * KP, g);
      const f32x4 s = row_mma(kf, qf, f32x4{0.f, 0.f, 0.f, 0.f});
      const f32x4 dp = row_mma(vf, dof, f32x4{0.f, 0.f, 0.f, 0.f});
      float ds[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = (s0 + 4 * g + i < ncq) ? fast_exp2(s[i] * a.scale_log2 - lse2) : 0.f;
        ds[i] = p * (dp[i] - D);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] = col_mma(Kt + (16 * t + r) * kTP + 16 * st + 4 * g, ds, acc[t]);
    }
  }
  if (qv) {
    T* p = static_cast<T*>(a.drq) + b * a.drq_sb + lh * a.drq_sh + (int64_t)qi * a.drq_sn;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int d = 16 * t + 4 * g;
      if (d < a.Ldh) {
        float v4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v4[i] = acc[t][i] * a.scale;
        store4<T>(p + d, v4);
      }
    }
  }
}

// ----------------------------------------------------------------------------
// backward pass KV: dgk / dgv partial sums of one 16-latent tile over one segment of queries
// ----------------------------------------------------------------------------
template <typename T, int DHP>
__global__ __launch_bounds__(256, DHP <= 32 ? 5 : 1) void latent_bwd_kv_kernel(const LatentArgs a) {
  constexpr int DQ = DHP / 4, NT = DHP / 16, KP = DHP + kRowPad<T>;
  __shared__ __align__(16) T Qs[64 * KP];
  __shared__ __align__(16) T Qt[DHP * kTP];
  __shared__ __align__(16) T Os[64 * KP];
  __shared__ __align__(16) T Ot[DHP * kTP];
  __shared__ __align__(16) T Rs[64 * KP];  // drq rows of the tile (wave w: rows 16 w .. 16 w + 15)
  __shared__ float lse2s[64], Dss[64];
  __shared__ int vis[64];
  static_assert(sizeof(T) * 64 * KP >= 2 * DHP * 16 * sizeof(float), "reduction buffer does not fit in Qs");
  float* red = reinterpret_cast<float*>(Qs);  // [2][DHP][16] after the query loop

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane & 15, g = lane >> 4;
  const int seg = blockIdx.x % a.n_seg, rest = blockIdx.x / a.n_seg;
  const int lt = rest % a.n_lt, bh = rest / a.n_lt, lh = bh % a.Lh, b = bh / a.Lh;
  const int n0 = lt * 16, kj = n0 + r;
  const bool kv = kj < a.n_chunks;
  const T* rqb = static_cast<const T*>(a.rq) + b * a.rq_sb + lh * a.rq_sh;
  const T* dlb = static_cast<const T*>(a.dout) + b * a.do_sb + lh * a.do_sh;
  const int64_t hrow = ((int64_t)b * a.Lh + lh) * a.n_q;

  RowFrag<T, DQ> kf, vf;
  kf.load(static_cast<const T*>(a.gk) + b * a.gk_sb + lh * a.gk_sh + (int64_t)kj * a.gk_sn, g, a.Ldh, kv);
  vf.load(static_cast<const T*>(a.gv) + b * a.gv_sb + lh * a.gv_sh + (int64_t)kj * a.gv_sn, g, a.Ldh, kv);
  f32x4 dk[NT], dv[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) dk[t] = dv[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // first query that sees latent n0: s * q_block >= (n0 + 1) * chunk
  const int64_t need = (int64_t)(n0 + 1) * a.chunk;
  const int s_first = (int)((need + a.q_block - 1) / a.q_block);
  const int qbeg = max(seg * a.seg, s_first);
  const int qend = (int)min((int64_t)(seg + 1) * a.seg, (int64_t)a.n_q);
  // kAhead: the next 64 query rows (lse / D raw, transformed when staged) load while the current tile is worked
  // on; only where the extra registers leave the waves per SIMD as they are (narrow latent heads)
  constexpr bool kAhead = DHP * sizeof(T) <= 64;
  TransTile<T, DHP> tq, to;
  float pl = 0.f, pd = 0.f;
  auto load_tile = [&](int q0) {
    tq.load(rqb, a.rq_sn, q0, qend, a.Ldh);
    to.load(dlb, a.do_sn, q0, qend, a.Ldh);
    if (tid < 64) {
      const int qi = min(q0 + tid, qend - 1);
      pl = a.lse[hrow + qi];
      pd = a.Dsum[hrow + qi];
    }
  };
  if (kAhead && qbeg < qend) load_tile(qbeg);
  for (int q0 = qbeg; q0 < qend; q0 += 64) {
    if (!kAhead) load_tile(q0);
    lds_barrier();
    tq.template store_rows<KP>(Qs);
    tq.store_t(Qt);
    to.template store_rows<KP>(Os);
    to.store_t(Ot);
    if (tid < 64) {
      const int qq = q0 + tid;
      const bool qv = qq < qend;
      lse2s[tid] = (qv && pl != kNegInf) ? pl * kLog2e : 0.f;
      Dss[tid] = qv ? pd : 0.f;
      vis[tid] = qv ? visible(qq, a) : 0;
    }
    if (kAhead && q0 + 64 < qend) load_tile(q0 + 64);
    lds_barrier();
    const int s0 = q0 + 16 * wave;  // each wave takes one 16-query sub-tile
    if (s0 < qend) {
      RowFrag<T, DQ> qf, of;
      qf.load_lds(Qs + (16 * wave + r) * KP, g);
      of.load_lds(Os + (16 * wave + r) * KP, g);
      const f32x4 s = row_mma(qf, kf, f32x4{0.f, 0.f, 0.f, 0.f});   // S[query 4g+i][latent r]
      const f32x4 dp = row_mma(of, vf, f32x4{0.f, 0.f, 0.f, 0.f});  // dP[query][latent]
      float p[4], ds[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ql = 16 * wave + 4 * g + i;
        p[i] = (kv && kj < vis[ql]) ? fast_exp2(s[i] * a.scale_log2 - lse2s[ql]) : 0.f;
        ds[i] = p[i] * (dp[i] - Dss[ql]);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        dv[t] = col_mma(Ot + (16 * t + r) * kTP + 16 * wave + 4 * g, p, dv[t]);
        dk[t] = col_mma(Qt + (16 * t + r) * kTP + 16 * wave + 4 * g, ds, dk[t]);
      }
    }
  }
  // sum the four waves in order: red[which][dim][latent]
  for (int w = 0; w < 4; ++w) {
    lds_barrier();
    if (wave == w) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 16 * t + 4 * g + i;
          float* rk = red + (0 * DHP + d) * 16 + r;
          float* rv = red + (1 * DHP + d) * 16 + r;
          *rk = (w == 0 ? 0.f : *rk) + dk[t][i] * a.scale;
          *rv = (w == 0 ? 0.f : *rv) + dv[t][i];
        }
    }
  }
  lds_barrier();
  float* part = a.part + ((((int64_t)b * a.Lh + lh) * a.n_seg + seg) * a.n_lt * 16) * 2 * a.Ldh;
  for (int idx = tid; idx < 16 * 2 * a.Ldh; idx += 256) {
    const int n = idx / (2 * a.Ldh), which = (idx / a.Ldh) % 2, d = idx % a.Ldh;
    part[(int64_t)(n0 + n) * 2 * a.Ldh + which * a.Ldh + d] = red[(which * DHP + d) * 16 + n];
  }
}

// ----------------------------------------------------------------------------
// backward in one pass, bf16, one latent tile (n_chunks <= 16: config 2's 16 latents).  One workgroup per
// (batch, latent head, segment of a.seg queries): gk / gv are staged once, and each 64-query tile of the
// segment is read once.  Per 16-query sub-tile a wave computes, with the queries in lanes (as pass Q), D and
// drq, and, with the latents in lanes (as pass KV), the segment's dgk / dgv sums -- the products of the two
// passes, without re-reading rq and dL or writing D to the workspace (where the first query that sees a
// latent starts a 64-query tile and the segments are the same, as at config 2 with 16 latents, the
// summation order is theirs too).  The next query tile loads while the current one is worked on.
// ----------------------------------------------------------------------------
template <int DHP>
__global__ __launch_bounds__(256) void latent_bwd_fused_kernel(const LatentArgs a) {
  using T = uint16_t;
  constexpr int DQ = DHP / 4, NT = DHP / 16, KP = DHP + kRowPad<T>;
  __shared__ __align__(16) T Ks[64 * KP];   // gk rows (rows >= n_chunks zero)
  __shared__ __align__(16) T Kt[DHP * kTP]; // gk transposed
  __shared__ __align__(16) T Vs[64 * KP];   // gv rows
  __shared__ __align__(16) T Qs[64 * KP];   // rq rows of the query tile
  __shared__ __align__(16) T Qt[DHP * kTP]; // rq transposed
  __shared__ __align__(16) T Os[64 * KP];   // dL rows
  __shared__ __align__(16) T Ot[DHP * kTP]; // dL transposed
  __shared__ __align__(16) T Rs[64 * KP];  // drq rows of the tile (wave w: rows 16 w .. 16 w + 15)
  __shared__ float lse2s[64], Dss[64];
  __shared__ int vis[64];
  static_assert(sizeof(T) * 64 * KP >= 2 * DHP * 16 * sizeof(float), "reduction buffer does not fit in Qs");
  float* red = reinterpret_cast<float*>(Qs);  // [2][DHP][16] after the query loop

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane & 15, g = lane >> 4;
  const int seg = blockIdx.x % a.n_seg, bh = blockIdx.x / a.n_seg, lh = bh % a.Lh, b = bh / a.Lh;
  const bool kv = r < a.n_chunks;  // this lane's latent (latents in lanes)
  const T* rqb = static_cast<const T*>(a.rq) + b * a.rq_sb + lh * a.rq_sh;
  const T* dlb = static_cast<const T*>(a.dout) + b * a.do_sb + lh * a.do_sh;
  const int64_t hrow = ((int64_t)b * a.Lh + lh) * a.n_q;
  const int qbeg = seg * a.seg, qend = (int)min((int64_t)(seg + 1) * a.seg, (int64_t)a.n_q);

  TransTile<T, DHP> tq, to;
  float pl = 0.f;
  auto load_tile = [&](int q0) {
    tq.load(rqb, a.rq_sn, q0, qend, a.Ldh);
    to.load(dlb, a.do_sn, q0, qend, a.Ldh);
    if (tid < 64) pl = a.lse[hrow + min(q0 + tid, qend - 1)];
  };
  {  // the latents and the first query tile in flight together
    TransTile<T, DHP> tk;
    RowTile<T, DHP> tv;
    tk.load(static_cast<const T*>(a.gk) + b * a.gk_sb + lh * a.gk_sh, a.gk_sn, 0, a.n_chunks, a.Ldh);
    tv.load(static_cast<const T*>(a.gv) + b * a.gv_sb + lh * a.gv_sh, a.gv_sn, 0, a.n_chunks, a.Ldh);
    load_tile(qbeg);
    tk.template store_rows<KP>(Ks);
    tk.store_t(Kt);
    tv.template store<KP>(Vs);
  }
  lds_barrier();
  RowFrag<T, DQ> kf, vf;  // latent r's rows, for both orientations
  kf.load_lds(Ks + r * KP, g);
  vf.load_lds(Vs + r * KP, g);
  f32x4 dk[NT], dv[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) dk[t] = dv[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // the drq rows of the previous tile's sub-tile, staged in this wave's LDS rows, as 16-byte chunks in row
  // order: a store writes whole rows (8 rows of 64 dims) instead of 16 rows x 8 bytes.  They are stored
  // before the next tile's loads are issued: a store between those loads and their first use would make the
  // compiler's wait there count it as well (one counter for loads and stores, which may retire out of order).
  T* dbase = static_cast<T*>(a.drq) + b * a.drq_sb + lh * a.drq_sh;
  auto flush_drq = [&](int q0p) {
    constexpr int CPR = DHP / 8;  // 16-byte chunks per row; 16 CPR is a multiple of 64
    static_assert((16 * CPR) % 64 == 0, "whole store instructions");
    const T* sr = Rs + 16 * wave * KP;
#pragma unroll
    for (int it = 0; it < 16 * CPR / 64; ++it) {
      const int idx = 64 * it + lane, rr = idx / CPR, c = idx % CPR, q = q0p + 16 * wave + rr;
      const uint4 x = *reinterpret_cast<const uint4*>(sr + rr * KP + 8 * c);
      if (q < qend && 8 * c < a.Ldh) *reinterpret_cast<uint4*>(dbase + (int64_t)q * a.drq_sn + 8 * c) = x;
    }
  };
  for (int q0 = qbeg; q0 < qend; q0 += 64) {
    lds_barrier();  // every wave is done with the previous tile
    tq.template store_rows<KP>(Qs);
    tq.store_t(Qt);
    to.template store_rows<KP>(Os);
    to.store_t(Ot);
    if (tid < 64) {
      const int qq = q0 + tid;
      const bool qv = qq < qend;
      lse2s[tid] = (qv && pl != kNegInf) ? pl * kLog2e : 0.f;
      vis[tid] = qv ? visible(qq, a) : 0;
    }
    if (q0 > qbeg) flush_drq(q0 - 64);
    if (q0 + 64 < qend) load_tile(q0 + 64);
    lds_barrier();
    const int sq = 16 * wave;  // this wave's 16-query sub-tile of the tile
    if (q0 + sq >= qend) continue;  // uniform
    RowFrag<T, DQ> qf, of;
    qf.load_lds(Qs + (sq + r) * KP, g);
    of.load_lds(Os + (sq + r) * KP, g);
    // ---- queries in lanes (pass Q): S^T[latent 4g+i][query r], D, dS, drq ----
    {
      const int ql = sq + r, qi = q0 + ql;
      const int ncq = vis[ql];
      const float lse2 = lse2s[ql];
      const f32x4 s = row_mma(kf, qf, f32x4{0.f, 0.f, 0.f, 0.f});
      const f32x4 dp = row_mma(vf, of, f32x4{0.f, 0.f, 0.f, 0.f});
      float D = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (4 * g + i < ncq) D += fast_exp2(s[i] * a.scale_log2 - lse2) * dp[i];
      D = sum_groups(D);
      float ds[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = (4 * g + i < ncq) ? fast_exp2(s[i] * a.scale_log2 - lse2) : 0.f;
        ds[i] = p * (dp[i] - D);
      }
      if (g == 0) Dss[ql] = D;  // read below by the lanes that hold this query's latents
      f32x4 acc[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] = col_mma(Kt + (16 * t + r) * kTP + 4 * g, ds, f32x4{0.f, 0.f, 0.f, 0.f});
      // drq: the sub-tile's 16 rows staged in this wave's LDS rows (a wave's LDS operations run in order: no
      // barrier), stored by flush_drq at the next step
      T* sr = Rs + sq * KP;
#pragma unroll
      for (int t = 0; t < NT; ++t)
        *reinterpret_cast<uint2*>(sr + r * KP + 16 * t + 4 * g) =
            make_uint2(pack_bf16x2(acc[t][0] * a.scale, acc[t][1] * a.scale),
                       pack_bf16x2(acc[t][2] * a.scale, acc[t][3] * a.scale));
    }
    // ---- latents in lanes (pass KV): S[query 4g+i][latent r], dgk / dgv over the sub-tile's queries ----
    {
      const f32x4 s = row_mma(qf, kf, f32x4{0.f, 0.f, 0.f, 0.f});
      const f32x4 dp = row_mma(of, vf, f32x4{0.f, 0.f, 0.f, 0.f});
      float p[4], ds[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ql = sq + 4 * g + i;
        p[i] = (kv && r < vis[ql]) ? fast_exp2(s[i] * a.scale_log2 - lse2s[ql]) : 0.f;
        ds[i] = p[i] * (dp[i] - Dss[ql]);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        dv[t] = col_mma(Ot + (16 * t + r) * kTP + sq + 4 * g, p, dv[t]);
        dk[t] = col_mma(Qt + (16 * t + r) * kTP + sq + 4 * g, ds, dk[t]);
      }
    }
  }
  if (qend > qbeg) flush_drq(qbeg + (qend - qbeg - 1) / 64 * 64);  // the last tile's drq rows
  // sum the four waves in order: red[which][dim][latent]
  for (int w = 0; w < 4; ++w) {
    lds_barrier();
    if (wave == w) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 16 * t + 4 * g + i;
          float* rk = red + (0 * DHP + d) * 16 + r;
          float* rv = red + (1 * DHP + d) * 16 + r;
          *rk = (w == 0 ? 0.f : *rk) + dk[t][i] * a.scale;
          *rv = (w == 0 ? 0.f : *rv) + dv[t][i];
        }
    }
  }
  lds_barrier();
  float* part = a.part + (((int64_t)b * a.Lh + lh) * a.n_seg + seg) * 16 * 2 * a.Ldh;
  for (int idx = tid; idx < 16 * 2 * a.Ldh; idx += 256) {
    const int n = idx / (2 * a.Ldh), which = (idx / a.Ldh) % 2, d = idx % a.Ldh;
    part[(int64_t)n * 2 * a.Ldh + which * a.Ldh + d] = red[(which * DHP + d) * 16 + n];
  }
}

// dgk / dgv [b][n][lh][d] = sum over segments (in order) of the partials; four dims per thread (the latent
// head dim is a multiple of 4, the partials' rows 16-byte aligned)
template <typename T>
__global__ __launch_bounds__(256) void latent_reduce_kernel(const LatentArgs a) {
  const int dq = a.Ldh / 4;
  const int64_t total = (int64_t)a.B * a.Lh * a.n_chunks * 2 * dq;
  const int64_t seg_stride = (int64_t)a.n_lt * 16 * 2 * a.Ldh;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    int64_t rest = idx;
    const int d = (int)(rest % dq) * 4; rest /= dq;
    const int which = rest % 2; rest /= 2;
    const int n = rest % a.n_chunks; rest /= a.n_chunks;
    const int lh = rest % a.Lh;
    const int b = rest / a.Lh;
    const float* p = a.part + ((int64_t)b * a.Lh + lh) * a.n_seg * seg_stride + (int64_t)n * 2 * a.Ldh +
                     which * a.Ldh + d;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < a.n_seg; ++k) {
      const float4 v = *reinterpret_cast<const float4*>(p + k * seg_stride);
      s[0] += v.x;
      s[1] += v.y;
      s[2] += v.z;
      s[3] += v.w;
    }
    T* out = which == 0 ? static_cast<T*>(a.dgk) + b * a.dgk_sb + lh * a.dgk_sh + (int64_t)n * a.dgk_sn + d
                        : static_cast<T*>(a.dgv) + b * a.dgv_sb + lh * a.dgv_sh + (int64_t)n * a.dgv_sn + d;
    store4<T>(out, s);
  }
}

namespace {

template <typename T, int DHP>
void launch(bool fwd, const LatentArgs& a, hipStream_t st) {
  if (fwd) {
    hipLaunchKernelGGL((latent_fwd_kernel<T, DHP>), dim3(a.B * a.Lh * a.n_qt), dim3(256), 0, st, a);
  } else {
    if (latent_one_pass(a.n_lt, std::is_same_v<T, uint16_t>, DHP)) {  // one latent tile: both passes in one
      hipLaunchKernelGGL((latent_bwd_fused_kernel<DHP <= 128 ? DHP : 128>), dim3(a.B * a.Lh * a.n_seg), dim3(256), 0,
                         st, a);
    } else {
      hipLaunchKernelGGL((latent_bwd_q_kernel<T, DHP>), dim3(a.B * a.Lh * a.n_qt), dim3(256), 0, st, a);
      hipLaunchKernelGGL((latent_bwd_kv_kernel<T, DHP>), dim3(a.B * a.Lh * a.n_lt * a.n_seg), dim3(256), 0, st, a);
    }
    const int64_t total = (int64_t)a.B * a.Lh * a.n_chunks * 2 * (a.Ldh / 4);
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 1024);
    hipLaunchKernelGGL((latent_reduce_kernel<T>), dim3(blocks), dim3(256), 0, st, a);
  }
}
template <typename T>
bool dispatch(int dhp, bool fwd, const LatentArgs& a, hipStream_t st) {
  switch (dhp) {
    case 32: launch<T, 32>(fwd, a, st); return true;
    case 64: launch<T, 64>(fwd, a, st); return true;
    case 96: launch<T, 96>(fwd, a, st); return true;
    case 128: launch<T, 128>(fwd, a, st); return true;
    case 256:  // bf16 only: the fp32 tiles of 256 dims exceed the LDS
      if constexpr (std::is_same_v<T, uint16_t>) {
        launch<T, 256>(fwd, a, st);
        return true;
      }
      return false;
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
  a->chunk = s->chunk; a->n_chunks = s->n_chunks;
  a->n_qt = (s->n_q + 63) / 64;
  a->n_lt = (s->n_chunks + 15) / 16;
  a->seg = latent_seg(s->B, s->Lh, s->n_chunks, s->n_q, latent_one_pass(a->n_lt, s->dtype == LLATTN_BF16,
                                                                   padded_head_dim(s->Ldh)));
  a->n_seg = (s->n_q + a->seg - 1) / a->seg;
  a->scale = 1.0f / sqrtf((float)s->Ldh);
  a->scale_log2 = a->scale * kLog2e;
  a->rq = rq->ptr; a->rq_sb = rq->sb; a->rq_sn = rq->sn; a->rq_sh = rq->sh;
  a->gk = gk->ptr; a->gk_sb = gk->sb; a->gk_sn = gk->sn; a->gk_sh = gk->sh;
  a->gv = gv->ptr; a->gv_sb = gv->sb; a->gv_sn = gv->sn; a->gv_sh = gv->sh;
  return LLATTN_OK;
}

}  // namespace

size_t latent_workspace_bytes(const llattn_shape* s) {
  auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
  const size_t n_lt = (s->n_chunks + 15) / 16;
  const int seg = latent_seg(s->B, s->Lh, s->n_chunks, s->n_q,
                             latent_one_pass((int)n_lt, s->dtype == LLATTN_BF16, padded_head_dim(s->Ldh)));
  const size_t n_seg = (s->n_q + seg - 1) / seg;
  return up((size_t)s->B * s->Lh * s->n_q * 4) + up((size_t)s->B * s->Lh * n_seg * n_lt * 16 * 2 * s->Ldh * 4);
}

}  // namespace llattn

using namespace llattn;

extern "C" int32_t llattn_latent_fwd(const llattn_shape* s, const llattn_tensor* rq, const llattn_tensor* gk,
                                     const llattn_tensor* gv, const llattn_tensor* out, float* lse, void* stream) {
  LatentArgs a;
  int32_t rc = common(s, rq, gk, gv, &a);
  if (rc) return rc;
  if ((rc = check_view("latent_out", out, s->dtype, true))) return rc;
  a.out = out->ptr; a.o_sb = out->sb; a.o_sn = out->sn; a.o_sh = out->sh;
  a.lse = lse;
  const int dhp = padded_head_dim(s->Ldh);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool ok = s->dtype == LLATTN_F32 ? dispatch<float>(dhp, true, a, st) : dispatch<uint16_t>(dhp, true, a, st);
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
  auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
  a.Dsum = static_cast<float*>(workspace);
  a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + up((size_t)s->B * s->Lh * s->n_q * 4));
  const int dhp = padded_head_dim(s->Ldh);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool ok = s->dtype == LLATTN_F32 ? dispatch<float>(dhp, false, a, st) : dispatch<uint16_t>(dhp, false, a, st);
  if (!ok) return fail(LLATTN_ERR_UNSUPPORTED, "latent head_dim %d unsupported", s->Ldh);
  return check_launch("llattn_latent_bwd");
}
