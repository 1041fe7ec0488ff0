// Windowed local attention with the fused gate epilogue, forward and backward,
// for gfx950 (64-wide waves, bf16/fp32 MFMA, LDS-staged key/value tiles).
//
// Semantics (reference models.py:232-305, 416-438): query i attends keys
// max(0, i-W, floor(i/bs)*bs - W + 1) <= j <= i-1 with scale 1/sqrt(Dh);
// a query without keys outputs 0.  The gate mixes the local output O with the
// remote row R of the token: w = sigmoid(g_l.O - g_r.R), y = w O + (1-w) R.
//
// Work decomposition: one 256-thread workgroup per (batch, head, tile of 64
// queries) [forward, dQ pass] or (batch, head, tile of 64 keys) [dK/dV pass];
// each of the four waves owns 16 rows of the tile.  Keys (resp. queries) are
// streamed through LDS in tiles of 64 and consumed in 16-row sub-tiles.
#include "llattn_abi.h"
#include "llattn_device.h"
#include "llattn_local.h"

#include <climits>
#include <mutex>

namespace llattn {


// ----------------------------------------------------------------------------
// forward: local attention + gate mix
//
// Every global access is a coalesced copy of whole head rows (16-byte chunks,
// consecutive lanes on consecutive chunks of a row) between HBM and a
// row-major LDS tile; MFMA operands are read from the tiles: row operands with
// ds_read_b128, column operands (V^T) with the transposing LDS read.
// ----------------------------------------------------------------------------
template <typename T, int DHP>
__global__ __launch_bounds__(256) void local_fwd_kernel(const LocalArgs a) {
  constexpr int DQ = DHP / 4, NT = DHP / 16, KP = DHP + kRowPad<T>;
  __shared__ __align__(16) T S0[64 * KP];  // query rows -> value rows -> remote rows -> y
  __shared__ __align__(16) T S1[64 * KP];  // key rows -> o_local
  __shared__ __align__(16) float gls[DHP], grs[DHP];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane & 15, g = lane >> 4;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = bid % a.n_qt, bh = bid / a.n_qt, h = bh % a.H, b = bh / a.H;
  const int T_ = a.T, Dh = a.Dh;
  const int q0 = qt * 64, qw = q0 + wave * 16, qi = qw + r, row = wave * 16 + r;
  const bool qv = qi < T_;

  const T* qbase = static_cast<const T*>(a.q) + b * a.q_sb + h * a.q_sh;
  const T* kbase = static_cast<const T*>(a.k) + b * a.k_sb + h * a.k_sh;
  const T* vbase = static_cast<const T*>(a.v) + b * a.v_sb + h * a.v_sh;
  const T* rbase = static_cast<const T*>(a.rem) + b * a.r_sb + h * a.r_sh;

  // every global read of the workgroup is issued before its first barrier
  const int kbeg = max(0, q0 - a.W);
  const int kend = min(T_, q0 + 64) - 1;  // exclusive
  const int qend = min(T_, q0 + 64);
  RowTile<T, DHP> qreg, kreg, vreg, rreg;
  qreg.load(qbase, a.q_st, q0, qend, Dh);
  kreg.load(kbase, a.k_st, kbeg, kend, Dh);
  vreg.load(vbase, a.v_st, kbeg, kend, Dh);
  rreg.load_div(rbase, a.r_sn, q0, qend, a.q_block, Dh);
  for (int d = tid; d < DHP; d += 256) {
    gls[d] = d < Dh ? a.gl[h * a.gate_hs + d] : 0.f;
    grs[d] = d < Dh ? a.gr[h * a.gate_hs + d] : 0.f;
  }
  qreg.template store<KP>(S0);
  kreg.template store<KP>(S1);
  lds_barrier();
  RowFrag<T, DQ> qf;
  qf.load_lds(S0 + row * KP, g);

  const int lo = qv ? key_lo(qi, a.W, a.bs) : INT_MAX;
  const int hi = qi - 1;
  float m_run = kNegInf, l_run = 0.f;
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int wlo = max(0, qw - a.W), whi = min(qw + 15, T_ - 1) - 1;  // keys any query of this wave may use
  for (int k0 = kbeg; k0 < kend; k0 += 64) {
    lds_barrier();  // S0 (queries / previous values) and S1 (previous keys) are free
    vreg.template store<KP>(S0);
    if (k0 != kbeg) kreg.template store<KP>(S1);
    lds_barrier();
    if (k0 + 64 < kend) {  // the next tile's loads overlap this tile's math
      kreg.load(kbase, a.k_st, k0 + 64, kend, Dh);
      vreg.load(vbase, a.v_st, k0 + 64, kend, Dh);
    }
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int s0 = k0 + 16 * st;
      if (s0 >= kend || s0 + 15 < wlo || s0 > whi) continue;  // uniform over the wave
      RowFrag<T, DQ> kf;
      kf.load_lds(S1 + (16 * st + r) * KP, g);
      const f32x4 s = row_mma(kf, qf, f32x4{0.f, 0.f, 0.f, 0.f});  // S^T[key 4g+i][query r]
      float sv[4], mloc = kNegInf;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = s0 + 4 * g + i;
        sv[i] = (j >= lo && j <= hi) ? s[i] * a.scale_log2 : kNegInf;
        mloc = fmaxf(mloc, sv[i]);
      }
      mloc = max_groups(mloc);
      const float m_new = fmaxf(m_run, mloc);
      const float mu = (m_new == kNegInf) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run - mu);
      float pv[4], ps = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pv[i] = fast_exp2(sv[i] - mu);
        ps += pv[i];
      }
      l_run = l_run * alpha + ps;
      m_run = m_new;
#pragma unroll
      for (int t = 0; t < NT; ++t) {  // O^T += V^T P^T, V^T read transposed from the value rows
        acc[t] *= alpha;
        acc[t] = col_mma_rm<KP>(S0 + (16 * st) * KP + 16 * t, pv, acc[t]);
      }
    }
  }
  lds_barrier();  // S0 / S1 free
  rreg.template store<KP>(S0);
  lds_barrier();

  // ---- epilogue: normalise, gate, mix; rows go back through LDS ----
  const float l = sum_groups(l_run);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  float o[NT][4], rv[NT][4];
  float sl = 0.f, sr = 0.f;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int d = 16 * t + 4 * g;
    Raw4<T> rr4;
    rr4.load(S0 + row * KP + d, true);
    rr4.get(rv[t]);
    const float4 gl4 = *reinterpret_cast<const float4*>(gls + d);
    const float4 gr4 = *reinterpret_cast<const float4*>(grs + d);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[t][i] = round_t<T>(acc[t][i] * inv);
    sl += o[t][0] * gl4.x + o[t][1] * gl4.y + o[t][2] * gl4.z + o[t][3] * gl4.w;
    sr += rv[t][0] * gr4.x + rv[t][1] * gr4.y + rv[t][2] * gr4.z + rv[t][3] * gr4.w;
  }
  sl = sum_groups(sl);
  sr = sum_groups(sr);
  const float mm = fmaxf(sl, sr);
  const float el = __expf(sl - mm), er = __expf(sr - mm);
  const float wl = el / (el + er), wr = er / (el + er);
#pragma unroll
  for (int t = 0; t < NT; ++t) {  // each lane overwrites exactly the remote elements it read
    const int d = 16 * t + 4 * g;
    float yv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) yv[i] = wl * o[t][i] + wr * rv[t][i];
    store4<T>(S0 + row * KP + d, yv);
    store4<T>(S1 + row * KP + d, o[t]);
  }
  // o_local, lse and w feed only the backward: a forward-only call passes null for them
  if (qv && g == 0) {
    const int64_t idx = ((int64_t)b * a.H + h) * T_ + qi;
    if (a.lse) a.lse[idx] = l > 0.f ? (m_run + __log2f(l)) * kLn2 : kNegInf;
    if (a.w) a.w[idx] = wl;
  }
  lds_barrier();
  store_tile<T, DHP, KP>(static_cast<T*>(a.y) + b * a.y_sb + h * a.y_sh, a.y_st, S0, q0, qend, Dh);
  if (a.ol) store_tile<T, DHP, KP>(static_cast<T*>(a.ol) + b * a.o_sb + h * a.o_sh, a.o_st, S1, q0, qend, Dh);
}

// ----------------------------------------------------------------------------
// backward pass 1 (query tiles): gate backward, dremote, dO_local, D = dO.O,
// gate partial sums, dQ
// ----------------------------------------------------------------------------
template <typename T, int DHP>
__global__ __launch_bounds__(256) void local_bwd_q_kernel(const LocalArgs a) {
  constexpr int DQ = DHP / 4, NT = DHP / 16, KP = DHP + kRowPad<T>;
  __shared__ __align__(16) T S0[64 * KP];  // dy -> dO_local (kept: dO rows)            | loop: key rows
  __shared__ __align__(16) T S1[64 * KP];  // o_local -> query rows                       | loop: value rows
  __shared__ __align__(16) T S2[64 * KP];  // remote -> dremote                           | epilogue: dq
  __shared__ float gsum[4][3][DHP];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane & 15, g = lane >> 4;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = bid % a.n_qt, bh = bid / a.n_qt, h = bh % a.H, b = bh / a.H;
  const int T_ = a.T, Dh = a.Dh;
  const int q0 = qt * 64, qw = q0 + wave * 16, qi = qw + r, row = wave * 16 + r;
  const bool qv = qi < T_;
  const int qend = min(T_, q0 + 64);
  const int64_t hrow = ((int64_t)b * a.H + h) * T_;
  const T* qbase = static_cast<const T*>(a.q) + b * a.q_sb + h * a.q_sh;
  const T* kbase = static_cast<const T*>(a.k) + b * a.k_sb + h * a.k_sh;
  const T* vbase = static_cast<const T*>(a.v) + b * a.v_sb + h * a.v_sh;

  // ---- phase 1: gate backward, in the accumulator layout (dims 16t+4g+i) ----
  RowTile<T, DHP> dyreg, olreg, rreg, qreg;
  dyreg.load(static_cast<const T*>(a.dy) + b * a.dy_sb + h * a.dy_sh, a.dy_st, q0, qend, Dh);
  olreg.load(static_cast<const T*>(a.ol) + b * a.o_sb + h * a.o_sh, a.o_st, q0, qend, Dh);
  rreg.load_div(static_cast<const T*>(a.rem) + b * a.r_sb + h * a.r_sh, a.r_sn, q0, qend, a.q_block, Dh);
  qreg.load(qbase, a.q_st, q0, qend, Dh);
  const float wq = qv ? a.w[hrow + qi] : 0.f;
  const float lse_nat = qv ? a.lse[hrow + qi] : kNegInf;
  dyreg.template store<KP>(S0);
  olreg.template store<KP>(S1);
  rreg.template store<KP>(S2);
  lds_barrier();

  const float* glp = a.gl + h * a.gate_hs;
  const float* grp = a.gr + h * a.gate_hs;
  float dyv[NT][4], olv[NT][4], rv[NT][4];
  float dot1 = 0.f;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int d = 16 * t + 4 * g;
    Raw4<T> x;
    x.load(S0 + row * KP + d, true); x.get(dyv[t]);
    x.load(S1 + row * KP + d, true); x.get(olv[t]);
    x.load(S2 + row * KP + d, true); x.get(rv[t]);
#pragma unroll
    for (int i = 0; i < 4; ++i) dot1 += dyv[t][i] * (olv[t][i] - rv[t][i]);
  }
  dot1 = sum_groups(dot1);
  const float delta = wq * (1.f - wq) * dot1;
  float Dq = 0.f;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int d = 16 * t + 4 * g;
    float gl4[4] = {0.f, 0.f, 0.f, 0.f}, gr4[4] = {0.f, 0.f, 0.f, 0.f};
    if (d < Dh) {
      load4<float>(glp + d, gl4);
      load4<float>(grp + d, gr4);
    }
    float dov[4], drv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dov[i] = round_t<T>(wq * dyv[t][i] + delta * gl4[i]);
      drv[i] = (1.f - wq) * dyv[t][i] - delta * gr4[i];
      Dq += dov[i] * olv[t][i];
    }
    store4<T>(S0 + row * KP + d, dov);  // in place over the dy elements this lane read
    store4<T>(S2 + row * KP + d, drv);  // in place over the remote elements
    // gate and dremote column partial sums over the 16 queries of this wave (rows past the end are 0)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float pl = sum_rows16_last(delta * olv[t][i]);
      const float pr = sum_rows16_last(-delta * rv[t][i]);
      const float pb = sum_rows16_last(drv[i]);
      if (r == 15) {
        gsum[wave][0][d + i] = pl;
        gsum[wave][1][d + i] = pr;
        gsum[wave][2][d + i] = pb;
      }
    }
  }
  Dq = sum_groups(Dq);
  if (qv && g == 0) a.Dsum[hrow + qi] = Dq;
  lds_barrier();  // dO / dremote tiles complete; o_local no longer needed
  qreg.template store<KP>(S1);
  store_tile<T, DHP, KP>(static_cast<T*>(a.dO) + ((int64_t)b * T_ * a.H + h) * Dh, (int64_t)a.H * Dh, S0, q0, qend,
                         Dh);
  store_tile<T, DHP, KP>(static_cast<T*>(a.dr) + b * a.dr_sb + h * a.dr_sh, a.dr_st, S2, q0, qend, Dh);
  {
    const int nrow = a.B * a.n_qt, prow = b * a.n_qt + qt;
    for (int idx = tid; idx < 3 * DHP; idx += 256) {
      const int which = idx / DHP, d = idx % DHP;
      if (d < Dh) {
        const float sum = gsum[0][which][d] + gsum[1][which][d] + gsum[2][which][d] + gsum[3][which][d];
        a.gpart[(((int64_t)h * 3 + which) * Dh + d) * nrow + prow] = sum;
      }
    }
  }
  // first key / value tile in flight while the fragments are read
  const int kbeg = max(0, q0 - a.W);
  const int kend = min(T_, q0 + 64) - 1;
  RowTile<T, DHP> kreg, vreg;
  kreg.load(kbase, a.k_st, kbeg, kend, Dh);
  vreg.load(vbase, a.v_st, kbeg, kend, Dh);
  lds_barrier();
  RowFrag<T, DQ> qf, dof;
  qf.load_lds(S1 + row * KP, g);
  dof.load_lds(S0 + row * KP, g);

  // ---- phase 2: dQ = scale * sum_j dS_ij k_j ----
  const float lse2 = (lse_nat == kNegInf) ? 0.f : lse_nat * kLog2e;
  const int lo = qv ? key_lo(qi, a.W, a.bs) : INT_MAX;
  const int hi = qi - 1;
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int wlo = max(0, qw - a.W), whi = min(qw + 15, T_ - 1) - 1;
  for (int k0 = kbeg; k0 < kend; k0 += 64) {
    lds_barrier();  // fragments read / previous tile consumed
    kreg.template store<KP>(S0);
    vreg.template store<KP>(S1);
    lds_barrier();
    if (k0 + 64 < kend) {
      kreg.load(kbase, a.k_st, k0 + 64, kend, Dh);
      vreg.load(vbase, a.v_st, k0 + 64, kend, Dh);
    }
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int s0 = k0 + 16 * st;
      if (s0 >= kend || s0 + 15 < wlo || s0 > whi) continue;
      RowFrag<T, DQ> kf, vf;
      kf.load_lds(S0 + (16 * st + r) * KP, g);
      vf.load_lds(S1 + (16 * st + r) * KP, g);
      const f32x4 s = row_mma(kf, qf, f32x4{0.f, 0.f, 0.f, 0.f});    // S^T[key][query]
      const f32x4 dp = row_mma(vf, dof, f32x4{0.f, 0.f, 0.f, 0.f});  // dP^T[key][query]
      float ds[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = s0 + 4 * g + i;
        const float p = (j >= lo && j <= hi) ? fast_exp2(s[i] * a.scale_log2 - lse2) : 0.f;
        ds[i] = p * (dp[i] - Dq);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] = col_mma_rm<KP>(S0 + (16 * st) * KP + 16 * t, ds, acc[t]);  // K^T dS^T
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    float v4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v4[i] = acc[t][i] * a.scale;
    store4<T>(S2 + row * KP + 16 * t + 4 * g, v4);  // S2 was last read before the loop's barriers
  }
  lds_barrier();
  store_tile<T, DHP, KP>(static_cast<T*>(a.dq) + b * a.dq_sb + h * a.dq_sh, a.dq_st, S2, q0, qend, Dh);
}

// ----------------------------------------------------------------------------
// backward pass 2 (key tiles): dK, dV.  Every key's contributions come from the
// queries j+1 .. j+W, all visited by the one workgroup that owns the key.
// ----------------------------------------------------------------------------
template <typename T, int DHP>
__global__ __launch_bounds__(256) void local_bwd_kv_kernel(const LocalArgs a) {
  constexpr int DQ = DHP / 4, NT = DHP / 16, KP = DHP + kRowPad<T>;
  __shared__ __align__(16) T SQ[64 * KP];  // key rows -> query rows -> dk
  __shared__ __align__(16) T SO[64 * KP];  // value rows -> dO rows -> dv
  __shared__ float lse2s[64], Dss[64];
  __shared__ int los[64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane & 15, g = lane >> 4;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int kt = bid % a.n_qt, bh = bid / a.n_qt, h = bh % a.H, b = bh / a.H;
  const int T_ = a.T, Dh = a.Dh;
  const int j0 = kt * 64, kw = j0 + wave * 16, kj = kw + r, row = wave * 16 + r;
  const bool kv = kj < T_;
  const int jend = min(T_, j0 + 64);
  const int64_t hrow = ((int64_t)b * a.H + h) * T_;

  const T* qbase = static_cast<const T*>(a.q) + b * a.q_sb + h * a.q_sh;
  const T* obase = static_cast<const T*>(a.dO) + (int64_t)b * T_ * a.H * Dh + (int64_t)h * Dh;
  const int64_t o_st = (int64_t)a.H * Dh;

  const int qbeg = j0 + 1;
  const int qend = (int)min((int64_t)T_, (int64_t)j0 + 64 + a.W);  // exclusive
  RowTile<T, DHP> qreg, oreg;
  float ls_r = 0.f, ds_r = 0.f;
  auto load_tile = [&](int q0) {
    qreg.load(qbase, a.q_st, q0, qend, Dh);
    oreg.load(obase, o_st, q0, qend, Dh);
    if (tid < 64 && q0 + tid < qend) {
      ls_r = a.lse[hrow + q0 + tid];
      ds_r = a.Dsum[hrow + q0 + tid];
    }
  };
  {
    RowTile<T, DHP> kreg, vreg;
    kreg.load(static_cast<const T*>(a.k) + b * a.k_sb + h * a.k_sh, a.k_st, j0, jend, Dh);
    vreg.load(static_cast<const T*>(a.v) + b * a.v_sb + h * a.v_sh, a.v_st, j0, jend, Dh);
    if (qbeg < qend) load_tile(qbeg);
    kreg.template store<KP>(SQ);
    vreg.template store<KP>(SO);
  }
  lds_barrier();
  RowFrag<T, DQ> kf, vf;
  kf.load_lds(SQ + row * KP, g);
  vf.load_lds(SO + row * KP, g);
  f32x4 dk[NT], dv[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) dk[t] = dv[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int wqlo = kw + 1, wqhi = (int)min((int64_t)T_ - 1, (int64_t)kw + 15 + a.W);
  for (int q0 = qbeg; q0 < qend; q0 += 64) {
    lds_barrier();
    qreg.template store<KP>(SQ);
    oreg.template store<KP>(SO);
    if (tid < 64) {
      const int qq = q0 + tid;
      const bool in = qq < qend;
      lse2s[tid] = (!in || ls_r == kNegInf) ? 0.f : ls_r * kLog2e;
      Dss[tid] = in ? ds_r : 0.f;
      los[tid] = in ? key_lo(qq, a.W, a.bs) : INT_MAX;
    }
    lds_barrier();
    if (q0 + 64 < qend) load_tile(q0 + 64);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int s0 = q0 + 16 * st;
      if (s0 >= qend || s0 + 15 < wqlo || s0 > wqhi) continue;
      RowFrag<T, DQ> qf, of;
      qf.load_lds(SQ + (16 * st + r) * KP, g);
      of.load_lds(SO + (16 * st + r) * KP, g);
      const f32x4 s = row_mma(qf, kf, f32x4{0.f, 0.f, 0.f, 0.f});   // S[query 4g+i][key r]
      const f32x4 dp = row_mma(of, vf, f32x4{0.f, 0.f, 0.f, 0.f});  // dP[query][key]
      float p[4], ds[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ql = 16 * st + 4 * g + i, qq = q0 + ql;
        const bool ok = kv && kj >= los[ql] && kj <= qq - 1;
        p[i] = ok ? fast_exp2(s[i] * a.scale_log2 - lse2s[ql]) : 0.f;
        ds[i] = p[i] * (dp[i] - Dss[ql]);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        dv[t] = col_mma_rm<KP>(SO + (16 * st) * KP + 16 * t, p, dv[t]);   // dV^T = dO^T P
        dk[t] = col_mma_rm<KP>(SQ + (16 * st) * KP + 16 * t, ds, dk[t]);  // dK^T = Q^T dS
      }
    }
  }
  lds_barrier();
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    float kv4[4], vv4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kv4[i] = dk[t][i] * a.scale;
      vv4[i] = dv[t][i];
    }
    store4<T>(SQ + row * KP + 16 * t + 4 * g, kv4);
    store4<T>(SO + row * KP + 16 * t + 4 * g, vv4);
  }
  lds_barrier();
  store_tile<T, DHP, KP>(static_cast<T*>(a.dk) + b * a.dk_sb + h * a.dk_sh, a.dk_st, SQ, j0, jend, Dh);
  store_tile<T, DHP, KP>(static_cast<T*>(a.dv) + b * a.dv_sb + h * a.dv_sh, a.dv_st, SO, j0, jend, Dh);
}

// ----------------------------------------------------------------------------
// fused backward for windows W <= 64, bf16: one workgroup walks a segment of
// query tiles of one (batch, head) in order.  With W <= 64 the keys of query
// tile qt lie in key tiles qt-1 and qt, and key tile qt gets its queries from
// query tiles qt and qt+1, so after step qt key tile qt-1 is complete.  Every
// row of q, k, v, dy, o_local and remote is read from HBM once per segment
// (plus one tile of halo at each end), dO never leaves LDS, and each output
// row is written once, through the wave's LDS staging rows (whole-row stores).
//
// The two roles work one tile apart, with ONE LDS barrier per step:
//   query waves 0-3: gate backward of tile qt+1 (8 threads per row, 2 rows per
//     thread: dO into LDS, D / lse / key bounds, dremote staged for a store
//     after the dQ, gate partial sums kept per thread in registers for the
//     segment), then dQ of tile qt over key tiles qt-1 and qt (16 queries per
//     wave);
//   key waves 4-7: stage q / k / v of tile qt+1 into LDS (prefetched one step
//     ahead), then the dK / dV contributions of tile qt's queries to key tiles
//     qt-1 (then complete and stored) and qt (kept in registers).
// q and dO are double-buffered by tile parity, k and v triple-buffered, so the
// tile being produced never overwrites one being read.  Different work on the
// two waves of each SIMD (VALU-heavy gate, LDS/MFMA-bound products) overlaps.
// The segment's last key tile needs the queries of the next segment's first
// tile: an extra step at the end adds their contributions (that tile's own
// outputs belong to the next segment).  Every step issues the same memory
// operations (masked lanes use out-of-range buffer offsets), so the compiler's
// vmcnt waits are exact.  No atomics: every output has one writer.
// ----------------------------------------------------------------------------
template <int DHP>
__global__ __launch_bounds__(512) void local_bwd_fused_kernel(const LocalArgs a, int seg_tiles) {
  using T = uint16_t;
  constexpr int DQ = DHP / 4, NT = DHP / 16, KP = DHP + kRowPad<T>, TILE = 64 * KP;
  constexpr int GS = DHP / 8, GV = GS / 4;  // gate layout: 8 threads per row, GS dims each, GV groups of 4
  __shared__ __align__(16) T SQ[2 * TILE];  // query rows by tile parity
  __shared__ __align__(16) T SO[2 * TILE];  // dO rows by tile parity
  __shared__ __align__(16) T SK[3 * TILE];  // key rows by tile index mod 3
  __shared__ __align__(16) T SV[3 * TILE];  // value rows by tile index mod 3
  __shared__ __align__(16) float gls[DHP], grs[DHP];
  __shared__ __align__(16) float lse2s[2][64], Dss[2][64];
  __shared__ __align__(16) int los[2][64];
  constexpr int SPP = DHP + 8;              // row pitch of the output staging rows
  __shared__ __align__(16) T SST[8 * 16 * SPP];  // per wave: 16 output rows on their way to HBM

  const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool qrole = wave < 4;
  const int w4 = wave & 3, row = w4 * 16 + r;  // query row (query waves) or key row (key waves)
  const int rtid = tid & 255;                  // thread index within the role
  const int n_seg = (a.n_qt + seg_tiles - 1) / seg_tiles;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int seg = bid % n_seg, bh = bid / n_seg, h = bh % a.H, b = bh / a.H;
  const int t0 = seg * seg_tiles, t1 = min(a.n_qt, t0 + seg_tiles);
  const int tlast = min(t1, a.n_qt - 1);  // the extra step runs when t1 < n_qt
  const int T_ = a.T, Dh = a.Dh;
  const int64_t hrow = ((int64_t)b * a.H + h) * T_;
  // row strides below 2^24 and (batch, head) slabs below 2^30 elements (checked by the launcher)
  const int q_st = (int)a.q_st, k_st = (int)a.k_st, v_st = (int)a.v_st, dy_st = (int)a.dy_st, o_st = (int)a.o_st;
  const int r_sn = (int)a.r_sn, dq_st = (int)a.dq_st, dk_st = (int)a.dk_st, dv_st = (int)a.dv_st, dr_st = (int)a.dr_st;
  auto slab = [&](const void* base, int st) { return make_rsrc(base, ((int64_t)(T_ - 1) * st + Dh) * 2); };
  // 4 values of a row as bf16 through a buffer store (offset past the extent: dropped)
  auto store4 = [&](__amdgpu_buffer_rsrc_t rs, uint32_t off, const float v[4]) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 x = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    __builtin_amdgcn_raw_buffer_store_b64(x, rs, off, 0, 0);
  };

  // The wave's 16 accumulator rows (lane (r, g) holds columns 16t + 4g .. 16t + 4g + 3 of row r for block
  // t < NT) times `sc`, as bf16, to rows grow0 .. grow0 + 15 of the output: staged through this wave's LDS
  // rows, then stored as 16-byte chunks in row order, so one store instruction writes whole rows (about
  // five rows of Dh 2 bytes each) instead of 16 rows x 64 bytes.  Rows past T_ (or all of them when !ok)
  // and columns past Dh store past the buffer extent (dropped).  The LDS operations of a wave run in order,
  // so the wave's own staging rows need no barrier.
  auto store_acc16 = [&](__amdgpu_buffer_rsrc_t rs, bool ok, int grow0, int st, const f32x4 (&v)[NT], float sc) {
    typedef int i32x4_t __attribute__((ext_vector_type(4)));
    // the lane's coordinates from the exec mask (mbcnt), recomputed here rather than kept live across the
    // callers' loops
    const int ln = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)), lr = ln & 15, lg = ln >> 4;
    T* sw = SST + wave * 16 * SPP;
#pragma unroll
    for (int t = 0; t < NT; ++t)
      *reinterpret_cast<uint2*>(sw + lr * SPP + 16 * t + 4 * lg) =
          make_uint2(pack_bf16x2(v[t][0] * sc, v[t][1] * sc), pack_bf16x2(v[t][2] * sc, v[t][3] * sc));
    constexpr int CPR = DHP / 8;  // 16-byte chunks per staged row; 16 CPR is a multiple of 64
    static_assert((16 * CPR) % 64 == 0, "whole store instructions");
#pragma unroll
    for (int it = 0; it < 16 * CPR / 64; ++it) {
      const int idx = 64 * it + ln, rr = idx / CPR, c = idx % CPR, grr = grow0 + rr;
      const uint4 x = *reinterpret_cast<const uint4*>(sw + rr * SPP + 8 * c);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4_t, x), rs,
                                             (ok && grr < T_ && 8 * c < Dh) ? (uint32_t)(grr * st + 8 * c) * 2u : kOffOOB,
                                             0, 0);
    }
  };

  for (int d = tid; d < DHP; d += 512) {
    gls[d] = d < Dh ? a.gl[h * a.gate_hs + d] : 0.f;
    grs[d] = d < Dh ? a.gr[h * a.gate_hs + d] : 0.f;
  }
  lds_barrier();  // the gate vectors are read by every query thread from the prologue on

  // ---- query role: gate backward of one tile (rows gr0 and gr0 + 32, 8 threads per row) ----
  const T* dybase = static_cast<const T*>(a.dy) + b * a.dy_sb + h * a.dy_sh;
  const T* olbase = static_cast<const T*>(a.ol) + b * a.o_sb + h * a.o_sh;
  const T* rbase = static_cast<const T*>(a.rem) + b * a.r_sb + h * a.r_sh;
  const float* wrow = a.w + hrow;
  const float* lrow = a.lse + hrow;
  const int gr0 = rtid >> 3, gd0 = (rtid & 7) * GS;
  const bool qb1 = a.q_block == 1;
  // A thread's GS dims of a row move as a 16-byte piece A and an 8-byte piece B.  GS = 12: a lane pair (even,
  // odd) owns dims [24p, 24p + 24); the even lane takes A = +0..7 and B = +8..11, the odd lane B = +12..15 and
  // A = +16..23 -- two instructions per row, and the pair's B pieces are one contiguous 16 bytes.  GS = 8:
  // A only; GS = 4: B only.
  const bool ev = (rtid & 1) == 0;
  const int dA = (GS == 12 && !ev) ? gd0 + 4 : gd0, dB = (GS == 12 && ev) ? gd0 + 8 : gd0;
  struct Piece { uint4 A; uint2 B; };
  Piece pdy[2], pol[2], prm[2];
  float pw[2], plse[2];
  // this thread's gate and dremote column partial sums (over the segment's rows it gates)
  float accl[GS], accr[GS], accb[GS];
  // pieces of the row at element offset `row` (ok: the row exists)
  auto ld_row = [&](const __amdgpu_buffer_rsrc_t& rs, int row, bool ok, Piece& p) {
    if constexpr (GS != 4) p.A = buf_ld16(rs, (ok && dA < Dh) ? (uint32_t)(row + dA) * 2u : kOffOOB);
    if constexpr (GS != 8) p.B = buf_ld8(rs, (ok && dB < Dh) ? (uint32_t)(row + dB) * 2u : kOffOOB);
  };
  auto unpack_row = [&](const Piece& p, float (&v)[GS]) {
    float a8[8], b4[4];
    if constexpr (GS != 4) {
      unpack_bf16x4(make_uint2(p.A.x, p.A.y), a8);
      unpack_bf16x4(make_uint2(p.A.z, p.A.w), a8 + 4);
    }
    if constexpr (GS != 8) unpack_bf16x4(p.B, b4);
#pragma unroll
    for (int e = 0; e < GS; ++e) {
      if constexpr (GS == 4) v[e] = b4[e];
      else if constexpr (GS == 8) v[e] = a8[e];
      else v[e] = ev ? (e < 8 ? a8[e] : b4[e - 8]) : (e < 4 ? b4[e] : a8[e - 4]);
    }
  };
  auto load_gate = [&](int qt) {  // dy / o_local / remote rows, w and lse of tile qt (zero past the end)
    const int q0 = qt * 64, qend = min(T_, q0 + 64), rows = qend - q0;
    const auto rdy = make_rsrc(dybase + (int64_t)q0 * dy_st, ((int64_t)(rows - 1) * dy_st + Dh) * 2);
    const auto rol = make_rsrc(olbase + (int64_t)q0 * o_st, ((int64_t)(rows - 1) * o_st + Dh) * 2);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int grow = gr0 + 32 * u, qi = q0 + grow;
      ld_row(rdy, grow * dy_st, true, pdy[u]);
      ld_row(rol, grow * o_st, true, pol[u]);
      if (qb1) {  // one remote row per token
        const auto rrm = make_rsrc(rbase + (int64_t)q0 * r_sn, ((int64_t)(rows - 1) * r_sn + Dh) * 2);
        ld_row(rrm, grow * r_sn, true, prm[u]);
      } else {  // one remote row per latent query of q_block tokens: rows counted from the tile's first one
        const int rq0 = q0 / a.q_block;
        const int rrel = (qi - rq0 * a.q_block) / a.q_block, rlast = (qend - 1) / a.q_block - rq0;
        const auto rrm = make_rsrc(rbase + (int64_t)rq0 * r_sn, ((int64_t)rlast * r_sn + Dh) * 2);
        ld_row(rrm, rrel * r_sn, qi < T_, prm[u]);
      }
      const int qc = min(qi, T_ - 1);  // always one load each (rows past the end are masked by the gate)
      pw[u] = wrow[qc];
      plse[u] = lrow[qc];
    }
  };
  auto gate = [&](int qt, const __amdgpu_buffer_rsrc_t& rdr) {  // gate backward of tile qt (prefetched rows)
    const bool full = qt < t1;  // the extra step's tile belongs to the next segment: no outputs of its own
    const int q0 = qt * 64, par = qt & 1;
    const int qb0 = q0 / a.bs, qr0 = q0 - qb0 * a.bs;  // block of the tile's first row (uniform)
    T* so = SO + par * TILE;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int grow = gr0 + 32 * u, qi = q0 + grow;
      const bool qv = qi < T_;
      const float wq = qv ? pw[u] : 0.f, lse_nat = qv ? plse[u] : kNegInf;
      float dyv[GS], olv[GS], rmv[GS];
      uint2 drp[GV];  // dremote of this thread's dims, bf16 pairs
      unpack_row(pdy[u], dyv);
      unpack_row(pol[u], olv);
      unpack_row(prm[u], rmv);
      float dot1 = 0.f;
#pragma unroll
      for (int e = 0; e < GS; ++e) dot1 += dyv[e] * (olv[e] - rmv[e]);
      dot1 = sum_lanes8(dot1);
      const float delta = wq * (1.f - wq) * dot1;
      float Dp = 0.f;
#pragma unroll
      for (int j = 0; j < GV; ++j) {
        const int d = gd0 + 4 * j;
        const float4 gl4 = *reinterpret_cast<const float4*>(gls + d);
        const float4 gr4 = *reinterpret_cast<const float4*>(grs + d);
        const float glv[4] = {gl4.x, gl4.y, gl4.z, gl4.w}, grv[4] = {gr4.x, gr4.y, gr4.z, gr4.w};
        float dov[4], drv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = 4 * j + i;
          dov[i] = wq * dyv[e] + delta * glv[i];
          drv[i] = (1.f - wq) * dyv[e] - delta * grv[i];
        }
        // dO_local rounded to bf16 once: the packed words go to LDS and their values feed D = dO.o_local
        const uint2 dop = make_uint2(pack_bf16x2(dov[0], dov[1]), pack_bf16x2(dov[2], dov[3]));
        unpack_bf16x4(dop, dov);
#pragma unroll
        for (int i = 0; i < 4; ++i) Dp += dov[i] * olv[4 * j + i];
        *reinterpret_cast<uint2*>(so + grow * KP + d) = dop;
        drp[j] = make_uint2(pack_bf16x2(drv[0], drv[1]), pack_bf16x2(drv[2], drv[3]));
        if (full) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            accl[4 * j + i] += delta * olv[4 * j + i];
            accr[4 * j + i] -= delta * rmv[4 * j + i];
            accb[4 * j + i] += qv ? drv[i] : 0.f;
          }
        }
      }
      // dremote: row gr0 + 32 u into row 8 u + lane / 8 of this wave's LDS staging rows (the wave's 16 rows
      // are 8 w .. 8 w + 7 and 32 + 8 w .. 32 + 8 w + 7 of the tile), stored by flush_dr after the dQ
      // products: a store issued between the loads of the next tile and their first use makes the
      // compiler's wait for that use count the store too (one counter for loads and stores, which may
      // retire out of order), and that wait then also covers loads issued after it
#pragma unroll
      for (int j = 0; j < GV; ++j)
        *reinterpret_cast<uint2*>(SST + (wave * 16 + 8 * u + (lane >> 3)) * SPP + gd0 + 4 * j) = drp[j];
      Dp = sum_lanes8(Dp);
      if ((rtid & 7) == 0) {
        Dss[par][grow] = qv ? Dp : 0.f;
        lse2s[par][grow] = (!qv || lse_nat == kNegInf) ? 0.f : lse_nat * kLog2e;
        // key_lo without a division: bs >= 64 (launcher), so row q0 + grow lies in the tile's first
        // block or the next one
        const int blk = (qb0 + (qr0 + grow >= a.bs)) * a.bs;
        los[par][grow] = qv ? max(max(0, qi - a.W), blk - a.W + 1) : INT_MAX;
      }
    }
  };

  // the dremote rows of tile qt that its gate staged in this wave's LDS rows, as 16-byte chunks in row order
  auto flush_dr = [&](int qt, const __amdgpu_buffer_rsrc_t& rdr) {
    typedef int i32x4_t __attribute__((ext_vector_type(4)));
    constexpr int CPR = DHP / 8;
    static_assert((16 * CPR) % 64 == 0, "whole store instructions");
    const bool okr = qt < t1;
    const int q0r = qt * 64;
    const T* sw = SST + wave * 16 * SPP;
#pragma unroll
    for (int it = 0; it < 16 * CPR / 64; ++it) {
      const int idx = 64 * it + lane, rr = idx / CPR, c = idx % CPR;
      const int qr = q0r + 8 * wave + (rr & 7) + 32 * (rr >> 3);
      const uint4 x = *reinterpret_cast<const uint4*>(sw + rr * SPP + 8 * c);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4_t, x), rdr,
                                             (okr && qr < T_ && 8 * c < Dh) ? (uint32_t)(qr * dr_st + 8 * c) * 2u : kOffOOB,
                                             0, 0);
    }
  };

  // ---- key role: q / k / v rows of one tile, staged through registers ----
  const T* qbase = static_cast<const T*>(a.q) + b * a.q_sb + h * a.q_sh;
  const T* kbase = static_cast<const T*>(a.k) + b * a.k_sb + h * a.k_sh;
  const T* vbase = static_cast<const T*>(a.v) + b * a.v_sb + h * a.v_sh;
  BufTile<DHP, 256> rq, rk, rv;
  auto load_tiles = [&](int qt) {  // zero past the sequence
    const int q0 = qt * 64, qend = min(T_, q0 + 64);
    rq.load(qbase, q_st, q0, qend, Dh, rtid);
    rk.load(kbase, k_st, q0, qend, Dh, rtid);
    rv.load(vbase, v_st, q0, qend, Dh, rtid);
  };
  auto store_tiles = [&](int qt) {
    rq.template store<KP>(SQ + (qt & 1) * TILE, rtid);
    rk.template store<KP>(SK + (qt % 3) * TILE, rtid);
    rv.template store<KP>(SV + (qt % 3) * TILE, rtid);
  };

  // ---- prologue: tile t0 staged and gated, keys of tile t0-1 staged ----
  if (qrole) {
#pragma unroll
    for (int e = 0; e < GS; ++e) accl[e] = accr[e] = accb[e] = 0.f;
    load_gate(t0);
    gate(t0, slab(static_cast<T*>(a.dr) + b * a.dr_sb + h * a.dr_sh, dr_st));
    flush_dr(t0, slab(static_cast<T*>(a.dr) + b * a.dr_sb + h * a.dr_sh, dr_st));
    load_gate(t0 + 1);
  } else {
    if (t0 > 0) {
      const int p0 = (t0 - 1) * 64;
      rk.load(kbase, k_st, p0, p0 + 64, Dh, rtid);
      rv.load(vbase, v_st, p0, p0 + 64, Dh, rtid);
      rk.template store<KP>(SK + ((t0 - 1) % 3) * TILE, rtid);
      rv.template store<KP>(SV + ((t0 - 1) % 3) * TILE, rtid);
    }
    load_tiles(t0);
    store_tiles(t0);
    load_tiles(t0 + 1);
  }
  lds_barrier();

  if (qrole) {
    const auto rdr = slab(static_cast<T*>(a.dr) + b * a.dr_sb + h * a.dr_sh, dr_st);
    const auto rdq = slab(static_cast<T*>(a.dq) + b * a.dq_sb + h * a.dq_sh, dq_st);
    for (int qt = t0; qt <= tlast; ++qt) {
      // gate of the next tile (its rows were prefetched last step), then the loads of the one after
      if (qt + 1 <= tlast) gate(qt + 1, rdr);
      load_gate(qt + 2);
      // ---- dQ = scale * sum_j dS_ij k_j over key tiles qt-1 and qt ----
      const bool full = qt < t1;
      const int par = qt & 1;
      const T* sq = SQ + par * TILE;
      const T* so = SO + par * TILE;
      const int qw = qt * 64 + w4 * 16, qi = qw + r;
      const bool qv = qi < T_;
      f32x4 dq[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) dq[t] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (full) {
        RowFrag<T, DQ> qf, dof;
        qf.load_lds(sq + row * KP, g);
        dof.load_lds(so + row * KP, g);
        const float lse2 = lse2s[par][row], Dq = Dss[par][row];
        const int lo = los[par][row], hi = qi - 1;
        const int wlo = max(0, qw - a.W), whi = min(qw + 15, T_ - 1) - 1;
        // one 16-key sub-step st of key tile kt
        auto substep = [&](int kt, int st) {
          const T* Ks = SK + ((kt + 3) % 3) * TILE;
          const T* Vs = SV + ((kt + 3) % 3) * TILE;
          const int s0 = kt * 64 + 16 * st;
          RowFrag<T, DQ> kf, vf;
          kf.load_lds(Ks + (16 * st + r) * KP, g);
          vf.load_lds(Vs + (16 * st + r) * KP, g);
          const f32x4 sv = row_mma(kf, qf, f32x4{0.f, 0.f, 0.f, 0.f});    // S^T[key][query]
          const f32x4 dp = row_mma(vf, dof, f32x4{0.f, 0.f, 0.f, 0.f});  // dP^T[key][query]
          float ds[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = s0 + 4 * g + i;
            const float p = fast_exp2(sv[i] * a.scale_log2 - lse2);
            ds[i] = ((j >= lo) & (j <= hi)) ? p * (dp[i] - Dq) : 0.f;
          }
          const i16x4 dsb = pack_bf16x4(ds);
#pragma unroll
          for (int t = 0; t < NT; ++t) dq[t] = col_mma_rm<KP>(Ks + (16 * st) * KP + 16 * t, dsb, dq[t]);
        };
        if (qt > 0) {
          // The keys [qw - W, qw + 15) of this wave's queries (W <= 64) lie in the five sub-steps w4 .. w4 + 4
          // of key tiles qt-1 and qt, both staged: run exactly those, without branches, so the products of one
          // sub-step can overlap the softmax of the next (keys outside the window are masked to zero)
#pragma unroll
          for (int i = 0; i < 5; ++i) {
            const int sidx = w4 + i;
            substep(qt - 1 + (sidx >> 2), sidx & 3);
          }
        } else {
#pragma unroll
          for (int st = 0; st < 4; ++st) {  // key tile 0 only (there is no tile -1)
            const int s0 = 16 * st;
            if (s0 + 15 < wlo || s0 > whi) continue;  // uniform over the wave
            substep(0, st);
          }
        }
      }
      if (qt + 1 <= tlast) flush_dr(qt + 1, rdr);
      // lane holds dQ[query qi][16t + 4g + i]
      store_acc16(rdq, full, qw, dq_st, dq, a.scale);
      lds_barrier();  // tile qt+1 is staged and gated; every wave is done with tile qt-1's buffers
    }
  } else {
    const auto rdk = slab(static_cast<T*>(a.dk) + b * a.dk_sb + h * a.dk_sh, dk_st);
    const auto rdv = slab(static_cast<T*>(a.dv) + b * a.dv_sb + h * a.dv_sh, dv_st);
    f32x4 pk[NT], pv[NT];  // partial dK / dV of this wave's keys of key tile qt-1
#pragma unroll
    for (int t = 0; t < NT; ++t) pk[t] = pv[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int qt = t0; qt <= tlast; ++qt) {
      // stage the next tile (prefetched last step), then the loads of the one after
      if (qt + 1 <= tlast) store_tiles(qt + 1);
      load_tiles(qt + 2);
      // ---- dK / dV of this wave's 16 keys of tiles qt-1 (if owned: then complete) and qt ----
      const bool full = qt < t1, own_prev = qt - 1 >= t0;
      const int par = qt & 1;
      const T* sq = SQ + par * TILE;
      const T* so = SO + par * TILE;
      const int q0 = qt * 64, qend = min(T_, q0 + 64);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const bool active = half == 0 ? own_prev : full;  // uniform
        const int kt = qt - 1 + half;
        const int kw = kt * 64 + w4 * 16, kj = kw + r;
        const bool kv = kj < T_;
        const int wqlo = kw + 1, wqhi = (int)min((int64_t)T_ - 1, (int64_t)kw + 15 + a.W);
        f32x4 dk[NT], dv[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          dk[t] = half == 0 ? pk[t] : f32x4{0.f, 0.f, 0.f, 0.f};
          dv[t] = half == 0 ? pv[t] : f32x4{0.f, 0.f, 0.f, 0.f};
        }
        if (active) {
          RowFrag<T, DQ> kf, vf;
          kf.load_lds(SK + ((kt + 3) % 3) * TILE + row * KP, g);
          vf.load_lds(SV + ((kt + 3) % 3) * TILE + row * KP, g);
#pragma unroll
          for (int st = 0; st < 4; ++st) {
            const int s0 = q0 + 16 * st;
            if (s0 >= qend || s0 + 15 < wqlo || s0 > wqhi) continue;  // uniform
            RowFrag<T, DQ> qf, of;
            qf.load_lds(sq + (16 * st + r) * KP, g);
            of.load_lds(so + (16 * st + r) * KP, g);
            const int ql = 16 * st + 4 * g;  // this lane's four queries (rows of the step's tile)
            const int4 lo4 = *reinterpret_cast<const int4*>(&los[par][ql]);
            const float4 l4 = *reinterpret_cast<const float4*>(&lse2s[par][ql]);
            const float4 D4 = *reinterpret_cast<const float4*>(&Dss[par][ql]);
            const int lov[4] = {lo4.x, lo4.y, lo4.z, lo4.w};
            const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, Dv[4] = {D4.x, D4.y, D4.z, D4.w};
            const f32x4 sv = row_mma(qf, kf, f32x4{0.f, 0.f, 0.f, 0.f});  // S[query 4g+i][key r]
            const f32x4 dp = row_mma(of, vf, f32x4{0.f, 0.f, 0.f, 0.f});  // dP[query][key]
            float pp[4], ds[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int qq = q0 + ql + i;
              const bool ok = kv & (kj >= lov[i]) & (kj <= qq - 1);  // no short circuit: plain selects
              const float p = fast_exp2(sv[i] * a.scale_log2 - lv[i]);
              pp[i] = ok ? p : 0.f;
              ds[i] = pp[i] * (dp[i] - Dv[i]);
            }
            const i16x4 ppb = pack_bf16x4(pp), dsb = pack_bf16x4(ds);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
              dv[t] = col_mma_rm<KP>(so + (16 * st) * KP + 16 * t, ppb, dv[t]);  // dV^T = dO^T P
              dk[t] = col_mma_rm<KP>(sq + (16 * st) * KP + 16 * t, dsb, dk[t]);  // dK^T = Q^T dS
            }
          }
        }
        if (half == 0) {  // key tile qt-1 is complete: lane holds dK / dV[key kj][16t + 4g + i]
          store_acc16(rdk, own_prev, kw, dk_st, dk, a.scale);
          store_acc16(rdv, own_prev, kw, dv_st, dv, 1.f);
        } else {
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            pk[t] = dk[t];
            pv[t] = dv[t];
          }
        }
      }
      lds_barrier();  // tile qt+1 is staged and gated; every wave is done with tile qt-1's buffers
    }
    // a segment that ends the sequence: its last key tile gets no more queries
    if (t1 == a.n_qt) {
      const int kw = (t1 - 1) * 64 + w4 * 16;
      store_acc16(rdk, true, kw, dk_st, pk, a.scale);
      store_acc16(rdv, true, kw, dv_st, pv, 1.f);
    }
  }
  // gate and dremote partials of the segment: the 32 row threads of each dim (two rows each) added in
  // order, through LDS that no wave reads any more (the key tiles: 3 x 256 x GS floats fit in SK)
  static_assert(3 * 256 * GS * 4 <= 3 * TILE * 2, "partials staging exceeds the key tiles");
  float* gacc = reinterpret_cast<float*>(SK);  // [l | r | b][256 threads][GS]
  if (qrole) {
#pragma unroll
    for (int e = 0; e < GS; ++e) {
      gacc[rtid * GS + e] = accl[e];
      gacc[(256 + rtid) * GS + e] = accr[e];
      gacc[(512 + rtid) * GS + e] = accb[e];
    }
  }
  lds_barrier();
  const int nrow = a.B * n_seg, prow = b * n_seg + seg;
  for (int idx = tid; idx < 3 * DHP; idx += 512) {
    const int which = idx / DHP, d = idx % DHP;
    if (d < Dh) {
      const int sg = d / GS, e = d % GS;
      float s = 0.f;
      for (int rr = 0; rr < 32; ++rr) s += gacc[(which * 256 + rr * 8 + sg) * GS + e];
      a.gpart[(((int64_t)h * 3 + which) * Dh + d) * nrow + prow] = s;
    }
  }
}

// Query tiles per workgroup of the fused backward: enough workgroups for one
// per CU (256) where the (batch, head) count allows, otherwise whole sequences.
int fused_seg_tiles(const LocalArgs& a) {
  const int bh = a.B * a.H;
  const int want = max(1, (256 + bh - 1) / bh);
  return max(2, (a.n_qt + want - 1) / want);
}

// Ordered sums of the partials part[h][which][d][row] (which 0: gate_l, 1: gate_r, 2: dremote columns):
// dgate_l / dgate_r per head ([H][Dh]) or, for a gate shared by the heads, summed over them too ([Dh]);
// dbr[h][d] (when requested) over the rows.  Blocks [0, 2 ng) take one gate output each: the 256 threads
// stride over its (head, row) partials, eight independent loads in flight per thread, and a fixed tree adds
// the threads' sums (a shared gate's output sums H x rows partials; one wave per output would wait on one
// load chain per head).  The blocks after them take four dremote columns each, one wave per column.
__global__ __launch_bounds__(256) void gate_reduce_kernel(const float* __restrict__ part, float* dgl, float* dgr,
                                                          float* dbr, int H, int Dh, int nrow, int per_head) {
  __shared__ float red[256];
  const int tid = threadIdx.x, lane = tid & 63;
  const int ng = per_head ? H * Dh : Dh;  // outputs per gate vector
  if ((int)blockIdx.x < 2 * ng) {
    const int o = blockIdx.x, which = o / ng, od = o % ng, d = od % Dh;
    const int h0 = per_head ? od / Dh : 0, nh = per_head ? 1 : H;
    const int n = nh * nrow;  // partials of this output: index i = (h - h0) nrow + row
    auto at = [&](int i) {
      const int hh = h0 + i / nrow, rr = i - (i / nrow) * nrow;
      return part[(((int64_t)hh * 3 + which) * Dh + d) * nrow + rr];
    };
    float s = 0.f;
    int i = tid;
    for (; i + 7 * 256 < n; i += 8 * 256) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = at(i + 256 * u);
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; i < n; i += 256) s += at(i);
    red[tid] = s;
    __syncthreads();
#pragma unroll
    for (int w = 128; w > 0; w >>= 1) {
      if (tid < w) red[tid] += red[tid + w];
      __syncthreads();
    }
    if (tid == 0) (which == 0 ? dgl : dgr)[od] = red[0];
    return;
  }
  const int od = (blockIdx.x - 2 * ng) * 4 + (tid >> 6);  // dremote column h Dh + d
  if (!dbr || od >= H * Dh) return;  // whole waves exit; no barrier follows
  const float* p = part + (((int64_t)(od / Dh) * 3 + 2) * Dh + od % Dh) * nrow;
  float s = 0.f;
  for (int i = lane; i < nrow; i += 64) s += p[i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) dbr[od] = s;
}

// ----------------------------------------------------------------------------
// host launchers
// ----------------------------------------------------------------------------
bool strides_fit_32bit(const LocalArgs& a) {
  const int64_t lim = int64_t(1) << 24;
  const bool st32 = a.q_st <= lim && a.k_st <= lim && a.v_st <= lim && a.dy_st <= lim && a.o_st <= lim &&
                    a.r_sn <= lim && a.dq_st <= lim && a.dk_st <= lim && a.dv_st <= lim && a.dr_st <= lim;
  // outputs (and, in the wide backward, inputs) are addressed with 32-bit byte offsets over a (batch, head)
  // slab of T rows
  const int64_t slab = int64_t(1) << 30;
  return st32 && (int64_t)a.T * a.dq_st < slab && (int64_t)a.T * a.dk_st < slab && (int64_t)a.T * a.dv_st < slab &&
         (int64_t)a.T * a.dr_st < slab && (int64_t)a.T * a.q_st < slab && (int64_t)a.T * a.k_st < slab &&
         (int64_t)a.T * a.v_st < slab && (int64_t)a.T * a.dy_st < slab && (int64_t)a.T * a.o_st < slab &&
         (int64_t)a.T * a.r_sn < slab && (int64_t)a.T * a.H * a.Dh < slab;
}

namespace {

template <typename T, int DHP>
void launch_fwd(const LocalArgs& a, hipStream_t stream) {
  if constexpr (std::is_same_v<T, uint16_t>) {
    if (fwd32(a, LLATTN_BF16, DHP)) {
      launch_fwd32(a, DHP, stream);
      return;
    }
  }
  hipLaunchKernelGGL((local_fwd_kernel<T, DHP>), dim3(a.B * a.H * a.n_qt), dim3(256), 0, stream, a);
}
// The fused one-pass backward covers bf16 with padded head dims up to 96,
// windows up to 64 (keys of a query tile span two key tiles), local blocks of
// at least 64 tokens (a tile spans at most two blocks), row strides
// below 2^24 elements (its buffer loads address a 64-row tile with 32-bit
// byte offsets) and output slabs of T rows below 2^30 elements.
bool fused_bwd(const LocalArgs& a, int dtype, int dhp) {
  return dtype == LLATTN_BF16 && dhp <= 96 && a.W <= 64 && a.bs >= 64 && strides_fit_32bit(a);
}

template <typename T, int DHP>
void launch_bwd(const LocalArgs& a, hipStream_t stream) {
  if constexpr (std::is_same_v<T, uint16_t> && DHP <= 96) {
    if (fused_bwd(a, LLATTN_BF16, DHP)) {
      const int seg_tiles = fused_seg_tiles(a);
      const int n_seg = (a.n_qt + seg_tiles - 1) / seg_tiles;
      hipLaunchKernelGGL((local_bwd_fused_kernel<DHP>), dim3(a.B * a.H * n_seg), dim3(512), 0, stream, a, seg_tiles);
      return;
    }
  }
  if constexpr (std::is_same_v<T, uint16_t>) {
    if (wide_bwd(a, LLATTN_BF16, DHP)) {
      launch_bwd_wide(a, DHP, stream);
      return;
    }
  }
  hipLaunchKernelGGL((local_bwd_q_kernel<T, DHP>), dim3(a.B * a.H * a.n_qt), dim3(256), 0, stream, a);
  hipLaunchKernelGGL((local_bwd_kv_kernel<T, DHP>), dim3(a.B * a.H * a.n_qt), dim3(256), 0, stream, a);
}

template <typename T>
bool dispatch(int dhp, bool fwd, const LocalArgs& a, hipStream_t s) {
  switch (dhp) {
    case 32: fwd ? launch_fwd<T, 32>(a, s) : launch_bwd<T, 32>(a, s); return true;
    case 64: fwd ? launch_fwd<T, 64>(a, s) : launch_bwd<T, 64>(a, s); return true;
    case 96: fwd ? launch_fwd<T, 96>(a, s) : launch_bwd<T, 96>(a, s); return true;
    case 128: fwd ? launch_fwd<T, 128>(a, s) : launch_bwd<T, 128>(a, s); return true;
    case 256:  // bf16 only: the fp32 tiles of 256 dims exceed the LDS
      if constexpr (std::is_same_v<T, uint16_t>) {
        fwd ? launch_fwd<T, 256>(a, s) : launch_bwd<T, 256>(a, s);
        return true;
      }
      return false;
    default: return false;
  }
}

void set_view(const llattn_tensor* t, const void** p, int64_t* sb, int64_t* sn, int64_t* sh) {
  *p = t->ptr;
  *sb = t->sb;
  *sn = t->sn;
  *sh = t->sh;
}
void set_view(const llattn_tensor* t, void** p, int64_t* sb, int64_t* sn, int64_t* sh) {
  *p = t->ptr;
  *sb = t->sb;
  *sn = t->sn;
  *sh = t->sh;
}

int32_t common_args(const llattn_shape* s, const llattn_tensor* q, const llattn_tensor* k, const llattn_tensor* v,
                    const llattn_tensor* remote, const float* gate_l, const float* gate_r, LocalArgs* a) {
  int32_t rc = check_shape(s);
  if (rc) return rc;
  if ((rc = check_view("q", q, s->dtype, true)) || (rc = check_view("k", k, s->dtype, true)) ||
      (rc = check_view("v", v, s->dtype, true)) || (rc = check_view("remote", remote, s->dtype, true)))
    return rc;
  if (!gate_l || !gate_r || !aligned16(gate_l) || !aligned16(gate_r))
    return fail(LLATTN_ERR_LAYOUT, "gate vectors must be non-null 16-byte aligned fp32 arrays");
  *a = LocalArgs{};
  a->B = s->B; a->T = s->T; a->H = s->H; a->Dh = s->Dh; a->W = s->window; a->bs = s->block;
  a->q_block = s->q_block; a->n_qt = (s->T + 63) / 64; a->gate_hs = s->gate_per_head ? s->Dh : 0;
  a->scale = 1.0f / sqrtf((float)s->Dh);
  a->scale_log2 = a->scale * kLog2e;
  set_view(q, &a->q, &a->q_sb, &a->q_st, &a->q_sh);
  set_view(k, &a->k, &a->k_sb, &a->k_st, &a->k_sh);
  set_view(v, &a->v, &a->v_sb, &a->v_st, &a->v_sh);
  set_view(remote, &a->rem, &a->r_sb, &a->r_sn, &a->r_sh);
  a->gl = gate_l;
  a->gr = gate_r;
  return LLATTN_OK;
}

}  // namespace
}  // namespace llattn

using namespace llattn;

extern "C" int32_t llattn_local_gate_fwd(const llattn_shape* s, const llattn_tensor* q, const llattn_tensor* k,
                                         const llattn_tensor* v, const llattn_tensor* remote, const float* gate_l,
                                         const float* gate_r, const llattn_tensor* y, const llattn_tensor* o_local,
                                         float* lse, float* w, void* stream) {
  LocalArgs a;
  int32_t rc = common_args(s, q, k, v, remote, gate_l, gate_r, &a);
  if (rc) return rc;
  if ((rc = check_view("y", y, s->dtype, true))) return rc;
  // forward only: o_local (null view or null pointer), lse and w may all be omitted together
  const bool infer = (!o_local || !o_local->ptr) && !lse && !w;
  if (!infer) {
    if ((rc = check_view("o_local", o_local, s->dtype, true))) return rc;
    if (!lse || !w) return fail(LLATTN_ERR_LAYOUT, "lse / w outputs must be non-null (or all of o_local, lse, w null)");
    set_view(o_local, &a.ol, &a.o_sb, &a.o_st, &a.o_sh);
  }
  set_view(y, &a.y, &a.y_sb, &a.y_st, &a.y_sh);
  a.lse = lse;
  a.w = w;
  const int dhp = padded_head_dim(s->Dh);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool ok = s->dtype == LLATTN_F32 ? dispatch<float>(dhp, true, a, st) : dispatch<uint16_t>(dhp, true, a, st);
  if (!ok) return fail(LLATTN_ERR_UNSUPPORTED, "head_dim %d unsupported", s->Dh);
  return check_launch("llattn_local_gate_fwd");
}

namespace llattn {
namespace {

// Scratch of llattn_local_gate_bwd_noalloc: one copy per GPU, held from module load until the
// process ends.  Host code never passes the array's name to a kernel (on the host it is only a
// stand-in for the symbol); it passes the device address that hipGetSymbolAddress returns for the
// current device.
static __device__ __align__(256) unsigned char scratch[LLATTN_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per device.
int32_t scratch_on_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(LLATTN_ERR_LAUNCH, "llattn_local_gate_bwd_noalloc: no current HIP device (or more than %d)",
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(LLATTN_ERR_LAUNCH, "llattn_local_gate_bwd_noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                  dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return LLATTN_OK;
}

// Argument checks and views of the backward; the scratch pointers are filled in by the caller.
int32_t bwd_args(const llattn_shape* s, const llattn_tensor* q, const llattn_tensor* k, const llattn_tensor* v,
                 const llattn_tensor* remote, const float* gate_l, const float* gate_r, const llattn_tensor* o_local,
                 const float* lse, const float* w, const llattn_tensor* dy, const llattn_tensor* dq,
                 const llattn_tensor* dk, const llattn_tensor* dv, const llattn_tensor* dremote, float* dgate_l,
                 float* dgate_r, LocalArgs* a) {
  int32_t rc = common_args(s, q, k, v, remote, gate_l, gate_r, a);
  if (rc) return rc;
  if ((rc = check_view("o_local", o_local, s->dtype, true)) || (rc = check_view("dy", dy, s->dtype, true)) ||
      (rc = check_view("dq", dq, s->dtype, true)) || (rc = check_view("dk", dk, s->dtype, true)) ||
      (rc = check_view("dv", dv, s->dtype, true)) || (rc = check_view("dremote", dremote, s->dtype, true)))
    return rc;
  if (!lse || !w || !dgate_l || !dgate_r) return fail(LLATTN_ERR_LAYOUT, "lse / w / dgate pointers must be non-null");
  set_view(o_local, &a->ol, &a->o_sb, &a->o_st, &a->o_sh);
  set_view(dy, &a->dy, &a->dy_sb, &a->dy_st, &a->dy_sh);
  set_view(dq, &a->dq, &a->dq_sb, &a->dq_st, &a->dq_sh);
  set_view(dk, &a->dk, &a->dk_sb, &a->dk_st, &a->dk_sh);
  set_view(dv, &a->dv, &a->dv_sb, &a->dv_st, &a->dv_sh);
  set_view(dremote, &a->dr, &a->dr_sb, &a->dr_st, &a->dr_sh);
  a->lse = const_cast<float*>(lse);
  a->w = const_cast<float*>(w);
  return LLATTN_OK;
}

size_t up256(size_t x) { return (x + 255) & ~size_t(255); }

// Gate partial rows: one per (batch, segment) from the fused kernel, one per (batch, 128-query group) from
// the wide-window kernels, one per (batch, query tile) otherwise.
int gate_rows(const LocalArgs& a, int dtype) {
  const int dhp = padded_head_dim(a.Dh);
  if (fused_bwd(a, dtype, dhp)) {
    const int seg_tiles = fused_seg_tiles(a);
    return a.B * ((a.n_qt + seg_tiles - 1) / seg_tiles);
  }
  return wide_bwd(a, dtype, dhp) ? wide_gate_rows(a) : a.B * a.n_qt;
}

// Launches the backward kernels and the ordered gate reduction; a.dO / a.Dsum / a.gpart are set.
int32_t launch_bwd_all(const llattn_shape* s, const LocalArgs& a, float* dgate_l, float* dgate_r,
                       float* dremote_colsum, hipStream_t st) {
  const int dhp = padded_head_dim(s->Dh);
  const bool ok =
      s->dtype == LLATTN_F32 ? dispatch<float>(dhp, false, a, st) : dispatch<uint16_t>(dhp, false, a, st);
  if (!ok) return fail(LLATTN_ERR_UNSUPPORTED, "head_dim %d unsupported", s->Dh);
  const int nrow = gate_rows(a, s->dtype);
  const int per_head = s->gate_per_head ? 1 : 0;
  const int ng = per_head ? s->H * s->Dh : s->Dh;
  const int blocks = 2 * ng + (dremote_colsum ? (s->H * s->Dh + 3) / 4 : 0);
  hipLaunchKernelGGL(gate_reduce_kernel, dim3(blocks), dim3(256), 0, st, a.gpart, dgate_l, dgate_r,
                     dremote_colsum, s->H, s->Dh, nrow, per_head);
  return LLATTN_OK;
}

}  // namespace
}  // namespace llattn

extern "C" int32_t llattn_local_gate_bwd(const llattn_shape* s, const llattn_tensor* q, const llattn_tensor* k,
                                         const llattn_tensor* v, const llattn_tensor* remote, const float* gate_l,
                                         const float* gate_r, const llattn_tensor* o_local, const float* lse,
                                         const float* w, const llattn_tensor* dy, const llattn_tensor* dq,
                                         const llattn_tensor* dk, const llattn_tensor* dv,
                                         const llattn_tensor* dremote, float* dgate_l, float* dgate_r,
                                         float* dremote_colsum, void* workspace, size_t workspace_bytes,
                                         void* stream) {
  LocalArgs a;
  int32_t rc = bwd_args(s, q, k, v, remote, gate_l, gate_r, o_local, lse, w, dy, dq, dk, dv, dremote, dgate_l,
                        dgate_r, &a);
  if (rc) return rc;
  const size_t need = llattn_workspace_size(s, LLATTN_WS_LOCAL_BWD);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return fail(LLATTN_ERR_WORKSPACE, "local backward needs %zu workspace bytes (got %zu)", need, workspace_bytes);
  char* ws = static_cast<char*>(workspace);
  const size_t n_do = up256((size_t)s->B * s->T * s->H * s->Dh * elem_size(s->dtype));
  const size_t n_d = up256((size_t)s->B * s->H * s->T * 4);
  a.dO = ws;
  a.Dsum = reinterpret_cast<float*>(ws + n_do);
  a.gpart = reinterpret_cast<float*>(ws + n_do + n_d);
  if ((rc = launch_bwd_all(s, a, dgate_l, dgate_r, dremote_colsum, static_cast<hipStream_t>(stream)))) return rc;
  return check_launch("llattn_local_gate_bwd");
}

// The scratch holds only what the chosen kernels read and write: the gate partials for the fused
// one-pass backward; dO_local and the row sums D as well for the two-kernel backward.  Every byte
// the kernels read is written earlier in the same call, so nothing is cleared between calls.
extern "C" int32_t llattn_local_gate_bwd_noalloc(const llattn_shape* s, const llattn_tensor* q,
                                                 const llattn_tensor* k, const llattn_tensor* v,
                                                 const llattn_tensor* remote, const float* gate_l,
                                                 const float* gate_r, const llattn_tensor* o_local, const float* lse,
                                                 const float* w, const llattn_tensor* dy, const llattn_tensor* dq,
                                                 const llattn_tensor* dk, const llattn_tensor* dv,
                                                 const llattn_tensor* dremote, float* dgate_l, float* dgate_r,
                                                 float* dremote_colsum, void* stream) {
  LocalArgs a;
  int32_t rc = bwd_args(s, q, k, v, remote, gate_l, gate_r, o_local, lse, w, dy, dq, dk, dv, dremote, dgate_l,
                        dgate_r, &a);
  if (rc) return rc;
  const bool fused = fused_bwd(a, s->dtype, padded_head_dim(s->Dh));
  const size_t n_do = fused ? 0 : up256((size_t)s->B * s->T * s->H * s->Dh * elem_size(s->dtype));
  const size_t n_d = fused ? 0 : up256((size_t)s->B * s->H * s->T * 4);
  const size_t n_g = up256((size_t)s->H * 3 * s->Dh * gate_rows(a, s->dtype) * 4);
  if (n_do + n_d + n_g > LLATTN_NOALLOC_SCRATCH_BYTES)
    return fail(LLATTN_ERR_WORKSPACE,
                "llattn_local_gate_bwd_noalloc: this shape needs %zu scratch bytes, more than the library's "
                "%zu; call llattn_local_gate_bwd with a workspace instead",
                n_do + n_d + n_g, (size_t)LLATTN_NOALLOC_SCRATCH_BYTES);
  void* base = nullptr;
  if ((rc = scratch_on_current_device(&base))) return rc;
  char* ws = static_cast<char*>(base);
  a.dO = fused ? nullptr : ws;
  a.Dsum = fused ? nullptr : reinterpret_cast<float*>(ws + n_do);
  a.gpart = reinterpret_cast<float*>(ws + n_do + n_d);
  if ((rc = launch_bwd_all(s, a, dgate_l, dgate_r, dremote_colsum, static_cast<hipStream_t>(stream)))) return rc;
  return check_launch("llattn_local_gate_bwd_noalloc");
}
