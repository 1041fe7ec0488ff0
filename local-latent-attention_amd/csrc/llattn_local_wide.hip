// Local attention on 32x32x16 bf16 MFMA products (reference models.py:232-305,
// 416-438, and the autograd of both): the forward for every window, and the
// backward for windows above 64.
//
// Backward.  With W > 64 a query's keys span up to W/64 + 1 key tiles, so the
// work is MFMA-shaped (10 Dh flops per (query, key) pair against a few bytes
// per row).  A one-pass backward would keep, for every key tile in flight, the
// partial dQ of the W/64 + 1 query tiles it feeds (147 KB of fp32 at W = 512,
// Dh = 64): more than LDS or the register file holds.  So two atomic-free
// kernels share the pairs:
//
//   query side (local_bwd_wq_kernel), one workgroup per (batch, head, 128
//   queries): the gate backward of its rows (dO_local, D = dO.o_local,
//   dremote, gate partial sums; dO and D to the workspace), then dQ over the
//   keys [q0 - W, q0 + 127).  Wave w owns queries [q0 + 32 w, +32) and walks
//   the 32-key sub-steps of every 64-key chunk the workgroup stages.
//
//   key side (local_bwd_wkv_kernel), one workgroup per (batch, head, 128
//   keys): dK and dV over the queries [j0 + 1, j0 + 128 + W) in 128-query
//   chunks.  Wave w owns keys [j0 + 32 w, +32) and walks the 32-query
//   sub-steps of every chunk.
//
// 32 rows per wave keep a wave within 168 registers up to head dims of 64 in
// the forward and the query-side kernel, and their query (and dO) tiles share
// LDS with the key / value buffers (the waves hold their query operands in
// registers before the key loop starts), so three or four workgroups share a
// CU: the prologue's global-load round trips of one workgroup overlap the
// products of the others.  This file is compiled with
// -amdgpu-mfma-vgpr-form: accumulators live in VGPRs and no AGPRs are used, so
// a wave's whole 256-register budget is usable and the loops carry no copies
// between register files.  At Dh = 64 the softmax arithmetic of a score (an
// FMA, a quarter-rate exp, the dS terms, the bf16 packing) costs about as many
// issue cycles as its products.
//
// Operand layouts of v_mfma_f32_32x32x16_bf16 (lane l, half h = l / 32):
// A lane l holds row l % 32, k = 8 h .. 8 h + 7; B lane l holds column l % 32,
// k = 8 h .. 8 h + 7; the accumulator element i of lane l is row
// 8 (i / 4) + 4 h + i % 4, column l % 32.  Scores are formed with the row
// index (keys in the forward and the query-side kernel, queries in the
// key-side one) as the contraction index of the following product, so P and
// dS leave their accumulators as B operands without any data movement: the k
// slots of product m (0, 1) are accumulator elements 8 m .. 8 m + 7, i.e. rows
// 16 m + 4 h + e % 4 + 8 (e / 4), and the matching A operand (K^T, V^T, Q^T,
// dO^T with that row order) comes from two transposing LDS reads.
#include "llattn_abi.h"
#include "llattn_device.h"
#include "llattn_local.h"

#include <climits>

namespace llattn {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

constexpr int kWideRows = 128;  // queries (query side) or keys (key side) per workgroup

__device__ __forceinline__ f32x16 mma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// A or B operand from a row-major LDS tile (pitch P): lane l takes row `row0 + l % 32`, dims d0 + 8 h .. +7.
template <int P>
__device__ __forceinline__ bf16x8 frag_rows(const uint16_t* tile, int row0, int d0) {
  const int lane = threadIdx.x & 63;
  return __builtin_bit_cast(bf16x8, ld16(tile + (row0 + (lane & 31)) * P + d0 + 8 * (lane >> 5)));
}

// A operand X^T of a product whose 16 contraction slots are the tile rows r0 + 4 h + e % 4 + 8 (e / 4)
// (e = 0..7) and whose operand row (lane l % 32) is tile column c0 + l % 32.  In a ds_read_b64_tr_b16 the
// 16 lanes of a group read a 4 x 16 block (lane j: row j / 4, columns 4 (j % 4) .. +3) and lane r receives
// column r of its four rows; groups 2 g' and 2 g' + 1 (h = g') cover columns c0 .. c0 + 31.
template <int P>
__device__ __forceinline__ bf16x8 frag_cols(const uint16_t* tile, int r0, int c0) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const uint16_t* p = tile + (r0 + 4 * (g >> 1) + (r >> 2)) * P + c0 + 16 * (g & 1) + 4 * (r & 3);
  const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4*)(p));
  const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4*)(p + 8 * P));
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// accumulator elements 8 m .. 8 m + 7 as a bf16 B operand
__device__ __forceinline__ bf16x8 pack8(const float (&v)[16], int m) {
  const uint4 u = make_uint4(pack_bf16x2(v[8 * m], v[8 * m + 1]), pack_bf16x2(v[8 * m + 2], v[8 * m + 3]),
                             pack_bf16x2(v[8 * m + 4], v[8 * m + 5]), pack_bf16x2(v[8 * m + 6], v[8 * m + 7]));
  return __builtin_bit_cast(bf16x8, u);
}

__device__ __forceinline__ void unpack8(uint4 x, float* o) {
  unpack_bf16x4(make_uint2(x.x, x.y), o);
  unpack_bf16x4(make_uint2(x.z, x.w), o + 4);
}

// sum over the 16 lanes l' = l (mod 4) of a wave, in every lane: rotations within each 16-lane row, then
// across the rows
__device__ __forceinline__ float sum_stride4(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x124, 0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// Block class of 32 queries [qa, qa + 32) against 32 keys [ka, ka + 32): 0 no pair in the window, 1 every
// pair inside (distance 1 .. W - 1, so the block-start rule cannot drop one), 2 per-element masks.
__device__ __forceinline__ int block_class(int qa, int ka, int W) {
  const int dmin = qa - (ka + 31), dmax = qa + 31 - ka;
  if (dmax < 1 || dmin > W) return 0;
  return (dmin >= 1 && dmax <= W - 1) ? 1 : 2;
}

// ----------------------------------------------------------------------------
// query side: gate backward + dQ
// ----------------------------------------------------------------------------
template <int DHP>
__global__ __launch_bounds__(256, DHP <= 64 ? 3 : 1) void local_bwd_wq_kernel(const LocalArgs a) {
  using T = uint16_t;
  constexpr int KP = DHP + 8, KS = DHP / 16, DB = DHP / 32, TILE = 64 * KP;
  constexpr int CD = DHP / 4, CV = CD / 8;  // gate layout: 4 threads per row, CD dims each
  // key rows [buf], value rows [2 + buf]; before the key loop the query rows [q0, q0 + 128) (SQ) and the
  // dO_local rows (SD), whose operands the waves then hold in registers; dQ (bf16) in SQ at the end
  __shared__ __align__(16) T SKV[4 * TILE];
  T* const SQ = SKV;
  T* const SD = SKV + 2 * TILE;
  __shared__ __align__(16) float gsum[4 * 3 * DHP];  // gate and dremote partial sums [wave][3][DHP]
  __shared__ __align__(16) float gls[DHP], grs[DHP];
  __shared__ __align__(16) float lse2s[kWideRows], Dss[kWideRows];
  __shared__ __align__(16) int los[kWideRows];

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, c32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_qg = (a.T + kWideRows - 1) / kWideRows;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int qg = bid % n_qg, bh = bid / n_qg, hd = bh % a.H, b = bh / a.H;
  const int T_ = a.T, Dh = a.Dh, W = a.W, q0 = qg * kWideRows;
  const int64_t hrow = ((int64_t)b * a.H + hd) * T_;
  // 32-bit strides (checked by the launcher)
  const int q_st = (int)a.q_st, k_st = (int)a.k_st, v_st = (int)a.v_st, dy_st = (int)a.dy_st, o_st = (int)a.o_st;
  const int r_sn = (int)a.r_sn, dr_st = (int)a.dr_st, dq_st = (int)a.dq_st, do_st = a.H * Dh;
  auto slab = [&](const void* base, int st, int rows) { return make_rsrc(base, ((int64_t)(rows - 1) * st + Dh) * 2); };

  const T* qbase = static_cast<const T*>(a.q) + b * a.q_sb + hd * a.q_sh;
  const T* kbase = static_cast<const T*>(a.k) + b * a.k_sb + hd * a.k_sh;
  const T* vbase = static_cast<const T*>(a.v) + b * a.v_sb + hd * a.v_sh;
  T* dobase = static_cast<T*>(a.dO) + ((int64_t)b * T_ * a.H + hd) * Dh;

  // ---- loads: gate rows, query rows, first key / value chunk ----
  const int kbeg = max(0, q0 - W), kend = min(T_, q0 + kWideRows) - 1;  // keys [kbeg, kend)
  const int nch = kend > kbeg ? (kend - kbeg + 63) / 64 : 0;
  // every load of the prologue is issued before the first LDS store waits for one: a single round trip
  BufTile<DHP, 256> tk, tv, tq0, tq1;
  if (nch > 0) {
    tk.load(kbase, k_st, kbeg, kend, Dh, tid);
    tv.load(vbase, v_st, kbeg, kend, Dh, tid);
  }
  tq0.load(qbase, q_st, q0, min(T_, q0 + 64), Dh, tid);
  tq1.load(qbase, q_st, q0 + 64, min(T_, q0 + kWideRows), Dh, tid);
  const int gr = tid >> 2, gd0 = (tid & 3) * CD;
  const auto rdy = slab(static_cast<const T*>(a.dy) + b * a.dy_sb + hd * a.dy_sh, dy_st, T_);
  const auto rol = slab(static_cast<const T*>(a.ol) + b * a.o_sb + hd * a.o_sh, o_st, T_);
  const int n_rem = (T_ + a.q_block - 1) / a.q_block;
  const auto rrm = slab(static_cast<const T*>(a.rem) + b * a.r_sb + hd * a.r_sh, r_sn, n_rem);
  uint4 pdy[2][CV], pol[2][CV], prm[2][CV];
  float pw[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int qi = q0 + gr + 64 * u;
    const bool qv = qi < T_;
    const int rrow = qv ? qi / a.q_block : 0;
#pragma unroll
    for (int j = 0; j < CV; ++j) {
      const int d = gd0 + 8 * j;
      const bool ok = qv && d < Dh;
      pdy[u][j] = buf_ld16(rdy, ok ? (uint32_t)(qi * dy_st + d) * 2u : kOffOOB);
      pol[u][j] = buf_ld16(rol, ok ? (uint32_t)(qi * o_st + d) * 2u : kOffOOB);
      prm[u][j] = buf_ld16(rrm, ok ? (uint32_t)(rrow * r_sn + d) * 2u : kOffOOB);
    }
    pw[u] = qv ? a.w[hrow + qi] : 0.f;
  }
  const float glv = tid < Dh ? a.gl[hd * a.gate_hs + tid] : 0.f;  // DHP <= 128: one dim per thread
  const float grv = tid < Dh ? a.gr[hd * a.gate_hs + tid] : 0.f;
  const int qt = q0 + tid;
  const float lv = tid < kWideRows && qt < T_ ? a.lse[hrow + qt] : kNegInf;
  tq0.template store<KP>(SQ, tid);
  tq1.template store<KP>(SQ + TILE, tid);
  if (tid < DHP) {
    gls[tid] = glv;
    grs[tid] = grv;
  }
  if (tid < kWideRows) {
    lse2s[tid] = lv == kNegInf ? 0.f : lv * kLog2e;
    los[tid] = qt < T_ ? key_lo(qt, W, a.bs) : INT_MAX;
  }
  lds_barrier();  // gate vectors

  // ---- gate backward: 4 threads per row, rows gr and gr + 64 ----
  float accl[CD], accr[CD], accb[CD];
#pragma unroll
  for (int e = 0; e < CD; ++e) accl[e] = accr[e] = accb[e] = 0.f;
  const auto rdr = slab(static_cast<T*>(a.dr) + b * a.dr_sb + hd * a.dr_sh, dr_st, T_);
  const auto rdo = make_rsrc(dobase, ((int64_t)(T_ - 1) * do_st + Dh) * 2);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int row = gr + 64 * u, qi = q0 + row;
    const bool qv = qi < T_;
    float dyv[CD], olv[CD], rmv[CD];
#pragma unroll
    for (int j = 0; j < CV; ++j) {
      unpack8(pdy[u][j], dyv + 8 * j);
      unpack8(pol[u][j], olv + 8 * j);
      unpack8(prm[u][j], rmv + 8 * j);
    }
    float dot1 = 0.f;
#pragma unroll
    for (int e = 0; e < CD; ++e) dot1 += dyv[e] * (olv[e] - rmv[e]);
    dot1 += __shfl_xor(dot1, 1);
    dot1 += __shfl_xor(dot1, 2);
    const float wq = pw[u], delta = wq * (1.f - wq) * dot1;
    float Dp = 0.f;
#pragma unroll
    for (int j = 0; j < CV; ++j) {
      float dov[8], drv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int e = 8 * j + i, d = gd0 + e;
        dov[i] = wq * dyv[e] + delta * gls[d];
        drv[i] = (1.f - wq) * dyv[e] - delta * grs[d];
        accl[e] += delta * olv[e];
        accr[e] -= delta * rmv[e];
        accb[e] += drv[i];
      }
      // dO_local rounded to bf16 once: the packed words go to LDS and HBM, their values feed D = dO.o_local
      const uint4 dop = make_uint4(pack_bf16x2(dov[0], dov[1]), pack_bf16x2(dov[2], dov[3]),
                                   pack_bf16x2(dov[4], dov[5]), pack_bf16x2(dov[6], dov[7]));
      unpack8(dop, dov);
#pragma unroll
      for (int i = 0; i < 8; ++i) Dp += dov[i] * olv[8 * j + i];
      const int d = gd0 + 8 * j;
      st16(SD + row * KP + d, dop);
      const bool ok = qv && d < Dh;
      typedef int i32x4_t __attribute__((ext_vector_type(4)));
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4_t, dop), rdo,
                                             ok ? (uint32_t)(qi * do_st + d) * 2u : kOffOOB, 0, 0);
      const uint4 drp = make_uint4(pack_bf16x2(drv[0], drv[1]), pack_bf16x2(drv[2], drv[3]),
                                   pack_bf16x2(drv[4], drv[5]), pack_bf16x2(drv[6], drv[7]));
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4_t, drp), rdr,
                                             ok ? (uint32_t)(qi * dr_st + d) * 2u : kOffOOB, 0, 0);
    }
    Dp += __shfl_xor(Dp, 1);
    Dp += __shfl_xor(Dp, 2);
    if ((tid & 3) == 0) {
      Dss[row] = qv ? Dp : 0.f;
      if (qv) a.Dsum[hrow + qi] = Dp;
    }
  }
  // gate and dremote partial sums of the 128 rows: over the 16 rows of each wave (lanes of equal tid % 4),
  // then over the four waves in order
#pragma unroll
  for (int e = 0; e < CD; ++e) {
    const float l = sum_stride4(accl[e]), r = sum_stride4(accr[e]), s = sum_stride4(accb[e]);
    if (lane < 4) {
      gsum[(wave * 3 + 0) * DHP + gd0 + e] = l;
      gsum[(wave * 3 + 1) * DHP + gd0 + e] = r;
      gsum[(wave * 3 + 2) * DHP + gd0 + e] = s;
    }
  }
  lds_barrier();  // dO rows, D, gate sums
  {
    const int nrow = a.B * n_qg, prow = b * n_qg + qg;
    for (int idx = tid; idx < 3 * DHP; idx += 256) {
      const int which = idx / DHP, d = idx % DHP;
      if (d < Dh) {
        const float s = gsum[(0 * 3 + which) * DHP + d] + gsum[(1 * 3 + which) * DHP + d] +
                        gsum[(2 * 3 + which) * DHP + d] + gsum[(3 * 3 + which) * DHP + d];
        a.gpart[(((int64_t)hd * 3 + which) * Dh + d) * nrow + prow] = s;
      }
    }
  }

  // ---- this wave's operands: Q^T and dO^T of its 32 queries (B operands), lse, D, key bounds ----
  const int qw = 32 * wave;  // first query row of the wave within the workgroup
  bf16x8 qf[KS], of[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qf[ks] = frag_rows<KP>(SQ, qw, 16 * ks);
    of[ks] = frag_rows<KP>(SD, qw, 16 * ks);
  }
  const int myrow = qw + c32;
  const float lse2 = lse2s[myrow], Dq = Dss[myrow];
  const int lo = los[myrow], hi = q0 + myrow - 1;
  f32x16 dq[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dq[db] = zero16();
  lds_barrier();  // query and dO rows read: the key / value buffers are free

  // ---- dQ = scale * sum_j dS_ij k_j over the 64-key chunks [kbeg, kend), two 32-key sub-steps each ----
  for (int ci = 0; ci < nch; ++ci) {
    const int c0 = kbeg + 64 * ci, buf = ci & 1;
    T* sk = SKV + buf * TILE;
    T* sv = SKV + (2 + buf) * TILE;
    tk.template store<KP>(sk, tid);
    tv.template store<KP>(sv, tid);
    lds_barrier();  // also: every wave is done with the chunk that used this buffer two steps ago
    if (ci + 1 < nch) {
      tk.load(kbase, k_st, c0 + 64, kend, Dh, tid);
      tv.load(vbase, v_st, c0 + 64, kend, Dh, tid);
    }
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int ka = c0 + 32 * sb;
      const int cls = block_class(q0 + qw, ka, W);  // uniform over the wave
      if (cls) {
        f32x16 s = zero16(), dp = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          s = mma32(frag_rows<KP>(sk, 32 * sb, 16 * ks), qf[ks], s);    // S^T[key][query]
          dp = mma32(frag_rows<KP>(sv, 32 * sb, 16 * ks), of[ks], dp);  // dP^T[key][query]
        }
        float ds[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) ds[i] = fast_exp2(s[i] * a.scale_log2 - lse2) * (dp[i] - Dq);
        if (cls == 2) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int j = ka + 8 * (i >> 2) + 4 * h + (i & 3);
            ds[i] = ((j >= lo) & (j <= hi)) ? ds[i] : 0.f;
          }
        }
        const bf16x8 d0 = pack8(ds, 0), d1 = pack8(ds, 1);
#pragma unroll
        for (int db = 0; db < DB; ++db) {  // K^T[dim][key] with the keys in accumulator-row order
          dq[db] = mma32(frag_cols<KP>(sk, 32 * sb, 32 * db), d0, dq[db]);
          dq[db] = mma32(frag_cols<KP>(sk, 32 * sb + 16, 32 * db), d1, dq[db]);
        }
      }
    }
  }

  // ---- dQ rows out, through the query tile for 16-byte row stores ----
  lds_barrier();  // every wave is done with the key / value buffers
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * db + 8 * j + 4 * h;
      *reinterpret_cast<uint2*>(SQ + myrow * KP + d) =
          make_uint2(pack_bf16x2(dq[db][4 * j] * a.scale, dq[db][4 * j + 1] * a.scale),
                     pack_bf16x2(dq[db][4 * j + 2] * a.scale, dq[db][4 * j + 3] * a.scale));
    }
  lds_barrier();
  T* dqbase = static_cast<T*>(a.dq) + b * a.dq_sb + hd * a.dq_sh;
  store_tile<T, DHP, KP>(dqbase, dq_st, SQ, q0, T_, Dh);
  store_tile<T, DHP, KP>(dqbase, dq_st, SQ + TILE, q0 + 64, T_, Dh);
}

// ----------------------------------------------------------------------------
// key side: dK, dV
// ----------------------------------------------------------------------------
// Two workgroups per CU up to head dims of 64; wider heads hold more accumulators (dK and dV: 2 DHP / 2 per
// lane) and run one per CU.
template <int DHP>
__global__ __launch_bounds__(256, DHP <= 64 ? 2 : 1) void local_bwd_wkv_kernel(const LocalArgs a) {
  using T = uint16_t;
  constexpr int KP = DHP + 8, KS = DHP / 16, DB = DHP / 32, TILE = 64 * KP;
  constexpr int CH = 128, NH = CH / 64, NSB = CH / 32;  // queries per chunk, 64-row halves, 32-query sub-steps
  // chunk buffer `buf`: query rows at [2 buf NH TILE, +NH TILE), dO rows after them; prologue: keys, values
  __shared__ __align__(16) T SQO[4 * NH * TILE];
  __shared__ __align__(16) float lse2s[2][CH], Dss[2][CH];  // Dss: -D, the dP accumulators' initial values

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, c32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_kg = (a.T + kWideRows - 1) / kWideRows;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int kg = bid % n_kg, bh = bid / n_kg, hd = bh % a.H, b = bh / a.H;
  const int T_ = a.T, Dh = a.Dh, W = a.W, bs = a.bs, j0 = kg * kWideRows;
  const int64_t hrow = ((int64_t)b * a.H + hd) * T_;
  const int q_st = (int)a.q_st, k_st = (int)a.k_st, v_st = (int)a.v_st, do_st = a.H * Dh;

  const T* qbase = static_cast<const T*>(a.q) + b * a.q_sb + hd * a.q_sh;
  const T* dobase = static_cast<const T*>(a.dO) + ((int64_t)b * T_ * a.H + hd) * Dh;

  // queries [qbeg, qend) see at least one of the keys [j0, j0 + 128)
  const int qbeg = j0 + 1, qend = (int)min((int64_t)T_, (int64_t)j0 + kWideRows + W);
  const int nch = qend > qbeg ? (qend - qbeg + CH - 1) / CH : 0;
  BufTile<DHP, 256> tq[NH], to[NH];
  float pl = 0.f, pd = 0.f;
  auto load_chunk = [&](int c0) {
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
      tq[hh].load(qbase, q_st, c0 + 64 * hh, qend, Dh, tid);
      to[hh].load(dobase, do_st, c0 + 64 * hh, qend, Dh, tid);
    }
    // raw values of a valid row (rows past qend are zeroed when staged): nothing here uses the loaded values,
    // so the loads stay in flight with the tiles' until the chunk is staged
    if (tid < CH) {
      const int qi = min(c0 + tid, qend - 1);
      pl = a.lse[hrow + qi];
      pd = a.Dsum[hrow + qi];
    }
  };
  // keys and values of the workgroup through LDS into this wave's B operands
  {  // the four key / value halves and the first query chunk in flight before the first LDS store waits
    BufTile<DHP, 256> t[4];
    const T* kbase = static_cast<const T*>(a.k) + b * a.k_sb + hd * a.k_sh;
    const T* vbase = static_cast<const T*>(a.v) + b * a.v_sb + hd * a.v_sh;
    t[0].load(kbase, k_st, j0, min(T_, j0 + 64), Dh, tid);
    t[1].load(kbase, k_st, j0 + 64, min(T_, j0 + kWideRows), Dh, tid);
    t[2].load(vbase, v_st, j0, min(T_, j0 + 64), Dh, tid);
    t[3].load(vbase, v_st, j0 + 64, min(T_, j0 + kWideRows), Dh, tid);
    if (nch > 0) load_chunk(qbeg);
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i].template store<KP>(SQO + i * TILE, tid);
  }
  lds_barrier();
  const int kw = 32 * wave;  // first key row of the wave within the workgroup
  bf16x8 kB[KS], vB[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    kB[ks] = frag_rows<KP>(SQO, kw, 16 * ks);
    vB[ks] = frag_rows<KP>(SQO + 2 * TILE, kw, 16 * ks);
  }
  const int kj = j0 + kw + c32;  // this lane's key (accumulator column)
  f32x16 dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dk[db] = dv[db] = zero16();
  lds_barrier();  // key / value rows read: the buffers take query chunks from here on

  for (int ci = 0; ci < nch; ++ci) {
    const int c0 = qbeg + CH * ci, buf = ci & 1;
    T* sq = SQO + 2 * buf * NH * TILE;
    T* so = sq + NH * TILE;
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
      tq[hh].template store<KP>(sq + hh * TILE, tid);
      to[hh].template store<KP>(so + hh * TILE, tid);
    }
    if (tid < CH) {
      const bool qv = c0 + tid < qend;
      lse2s[buf][tid] = (qv && pl != kNegInf) ? pl * kLog2e : 0.f;
      Dss[buf][tid] = qv ? -pd : 0.f;
    }
    lds_barrier();  // also: every wave is done with the chunk that used this buffer two steps ago
    if (ci + 1 < nch) load_chunk(c0 + CH);
    // the first query of a local block has one key fewer (reference models.py:249-292): bs >= W > 64, so a
    // chunk of CH queries holds at most CH / 64 block starts, the first at nb0
    const int nb0 = (c0 + bs - 1) / bs * bs, nb1 = nb0 + bs;
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
      const int cls = block_class(c0 + 32 * sb, j0 + kw, W);  // uniform over the wave
      if (cls == 0) continue;
      // this lane's 16 queries are accumulator rows 8 (i / 4) + 4 h + i % 4; the dP accumulator starts at
      // -D of its query, so it ends as dP - D
      f32x16 sc = zero16(), dpc;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float4 d4 = *reinterpret_cast<const float4*>(&Dss[buf][32 * sb + 8 * jj + 4 * h]);
        dpc[4 * jj] = d4.x;
        dpc[4 * jj + 1] = d4.y;
        dpc[4 * jj + 2] = d4.z;
        dpc[4 * jj + 3] = d4.w;
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        sc = mma32(frag_rows<KP>(sq, 32 * sb, 16 * ks), kB[ks], sc);   // S[query][key]
        dpc = mma32(frag_rows<KP>(so, 32 * sb, 16 * ks), vB[ks], dpc);  // dP[query][key] - D[query]
      }
      float p[16], ds[16];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float4 l4 = *reinterpret_cast<const float4*>(&lse2s[buf][32 * sb + 8 * jj + 4 * h]);
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int i = 4 * jj + c;
          p[i] = fast_exp2(sc[i] * a.scale_log2 - lv[c]);
          ds[i] = p[i] * dpc[i];
        }
      }
      if (cls == 2) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int qq = c0 + 32 * sb + 8 * (i >> 2) + 4 * h + (i & 3), dd = qq - kj;
          const bool ok = (dd >= 1) & (dd <= W - ((qq == nb0) | (qq == nb1)));
          p[i] = ok ? p[i] : 0.f;
          ds[i] = ok ? ds[i] : 0.f;
        }
      }
      const bf16x8 p0 = pack8(p, 0), p1 = pack8(p, 1), d0 = pack8(ds, 0), d1 = pack8(ds, 1);
#pragma unroll
      for (int db = 0; db < DB; ++db) {  // dV^T = dO^T P, dK^T = Q^T dS (queries in accumulator-row order)
        dv[db] = mma32(frag_cols<KP>(so, 32 * sb, 32 * db), p0, dv[db]);
        dv[db] = mma32(frag_cols<KP>(so, 32 * sb + 16, 32 * db), p1, dv[db]);
        dk[db] = mma32(frag_cols<KP>(sq, 32 * sb, 32 * db), d0, dk[db]);
        dk[db] = mma32(frag_cols<KP>(sq, 32 * sb + 16, 32 * db), d1, dk[db]);
      }
    }
  }

  // ---- rows out: lane (c32, h) holds dims 32 db + 8 j + 4 h .. +3 of key kj.  The wave's 32 dK and 32 dV
  // rows go through its own LDS rows (after a barrier: every wave is done with the query chunks), then out
  // as 16-byte chunks in row order, so a store writes whole rows instead of 32 rows x 8 bytes ----
  lds_barrier();
  T* sk = SQO + kw * KP;                // dK rows of the wave: rows kw .. kw + 31
  T* sv = SQO + (kWideRows + kw) * KP;  // dV rows
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * db + 8 * j + 4 * h;
      *reinterpret_cast<uint2*>(sk + c32 * KP + d) =
          make_uint2(pack_bf16x2(dk[db][4 * j] * a.scale, dk[db][4 * j + 1] * a.scale),
                     pack_bf16x2(dk[db][4 * j + 2] * a.scale, dk[db][4 * j + 3] * a.scale));
      *reinterpret_cast<uint2*>(sv + c32 * KP + d) =
          make_uint2(pack_bf16x2(dv[db][4 * j], dv[db][4 * j + 1]), pack_bf16x2(dv[db][4 * j + 2], dv[db][4 * j + 3]));
    }
  typedef int i32x4_t __attribute__((ext_vector_type(4)));
  const auto rdk = make_rsrc(static_cast<T*>(a.dk) + b * a.dk_sb + hd * a.dk_sh,
                             ((int64_t)(T_ - 1) * a.dk_st + Dh) * 2);
  const auto rdv = make_rsrc(static_cast<T*>(a.dv) + b * a.dv_sb + hd * a.dv_sh,
                             ((int64_t)(T_ - 1) * a.dv_st + Dh) * 2);
  const int dk_st = (int)a.dk_st, dv_st = (int)a.dv_st;
  constexpr int CPR = DHP / 8;  // 16-byte chunks per row; 32 CPR is a multiple of 64
  static_assert((32 * CPR) % 64 == 0, "whole store instructions");
#pragma unroll
  for (int it = 0; it < 32 * CPR / 64; ++it) {
    const int idx = 64 * it + lane, rr = idx / CPR, c = idx % CPR, key = j0 + kw + rr;
    const bool ok = key < T_ && 8 * c < Dh;
    const uint4 xk = *reinterpret_cast<const uint4*>(sk + rr * KP + 8 * c);
    const uint4 xv = *reinterpret_cast<const uint4*>(sv + rr * KP + 8 * c);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4_t, xk), rdk,
                                           ok ? (uint32_t)(key * dk_st + 8 * c) * 2u : kOffOOB, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4_t, xv), rdv,
                                           ok ? (uint32_t)(key * dv_st + 8 * c) * 2u : kOffOOB, 0, 0);
  }
}

// ----------------------------------------------------------------------------
// forward: local attention + gate mix (every window, bf16, padded head dims up to 128)
//
// One workgroup per (batch, head, 128 queries); wave w owns queries
// [q0 + 32 w, +32) and keeps S^T = K Q^T for each 32-key sub-step in one
// accumulator (lane = query, so the online-softmax statistics of a query live
// in one lane pair), then O^T += V^T P^T with P^T passed on as the B operand
// as in the backward.  The gate epilogue reads the remote rows staged in LDS
// and writes y and o_local through LDS for 16-byte row stores.
// ----------------------------------------------------------------------------
template <int DHP>
__global__ __launch_bounds__(256, DHP <= 64 ? 3 : 2) void local_fwd32_kernel(const LocalArgs a) {
  using T = uint16_t;
  constexpr int KP = DHP + 8, KS = DHP / 16, DB = DHP / 32, TILE = 64 * KP;
  // key rows [buf], value rows [2 + buf]; before the key loop the query rows (SQ, tiles 0 and 1), whose
  // operands the waves then hold in registers; in the epilogue the remote rows, replaced in place by the
  // y rows, in SQ and the o_local rows in tiles 2 and 3
  __shared__ __align__(16) T SKV[4 * TILE];
  T* const SQ = SKV;
  __shared__ __align__(16) float gls[DHP], grs[DHP];

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, c32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_qg = (a.T + kWideRows - 1) / kWideRows;
  // heads vary fastest: the workgroups that run together (one contiguous range per XCD) read whole token
  // rows of the packed q|k|v projection rather than one head's 2 Dh-byte slice of each row
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int hd = bid % a.H, rq = bid / a.H, qg = rq % n_qg, b = rq / n_qg;
  const int T_ = a.T, Dh = a.Dh, W = a.W, q0 = qg * kWideRows;
  const int k_st = (int)a.k_st, v_st = (int)a.v_st;
  const T* kbase = static_cast<const T*>(a.k) + b * a.k_sb + hd * a.k_sh;
  const T* vbase = static_cast<const T*>(a.v) + b * a.v_sb + hd * a.v_sh;
  const T* rbase = static_cast<const T*>(a.rem) + b * a.r_sb + hd * a.r_sh;
  const int r_sn = (int)a.r_sn;

  const int kbeg = max(0, q0 - W), kend = min(T_, q0 + kWideRows) - 1;  // keys [kbeg, kend)
  const int nch = kend > kbeg ? (kend - kbeg + 63) / 64 : 0;
  BufTile<DHP, 256> tk, tv;
  if (nch > 0) {
    tk.template load<kStream>(kbase, k_st, kbeg, kend, Dh, tid);
    tv.template load<kStream>(vbase, v_st, kbeg, kend, Dh, tid);
  }
  {  // both query halves and the gate vectors in flight before the first LDS store waits for them
    const T* qbase = static_cast<const T*>(a.q) + b * a.q_sb + hd * a.q_sh;
    BufTile<DHP, 256> tq0, tq1;
    tq0.template load<kStream>(qbase, (int)a.q_st, q0, min(T_, q0 + 64), Dh, tid);
    tq1.template load<kStream>(qbase, (int)a.q_st, q0 + 64, min(T_, q0 + kWideRows), Dh, tid);
    const float glv = tid < Dh ? a.gl[hd * a.gate_hs + tid] : 0.f;  // DHP <= 128: one dim per thread
    const float grv = tid < Dh ? a.gr[hd * a.gate_hs + tid] : 0.f;
    tq0.template store<KP>(SQ, tid);
    tq1.template store<KP>(SQ + TILE, tid);
    if (tid < DHP) {
      gls[tid] = glv;
      grs[tid] = grv;
    }
  }
  lds_barrier();
  const int qw = 32 * wave, myrow = qw + c32, qi = q0 + myrow;  // this lane's query (accumulator column)
  bf16x8 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qf[ks] = frag_rows<KP>(SQ, qw, 16 * ks);
  lds_barrier();  // query rows read: the key / value buffers are free
  const int lo = qi < T_ ? key_lo(qi, W, a.bs) : INT_MAX, hi = qi - 1;
  float m_run = kNegInf, l_run = 0.f;  // l_run: this lane's half of the row sum
  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = zero16();

  for (int ci = 0; ci < nch; ++ci) {
    const int c0 = kbeg + 64 * ci, buf = ci & 1;
    T* sk = SKV + buf * TILE;
    T* sv = SKV + (2 + buf) * TILE;
    tk.template store<KP>(sk, tid);
    tv.template store<KP>(sv, tid);
    lds_barrier();  // also: every wave is done with the chunk that used this buffer two steps ago
    if (ci + 1 < nch) {
      tk.template load<kStream>(kbase, k_st, c0 + 64, kend, Dh, tid);
      tv.template load<kStream>(vbase, v_st, c0 + 64, kend, Dh, tid);
    } else {  // the last chunk: the epilogue's remote rows of both query halves, in the key / value registers
      tk.load_div(rbase, r_sn, q0, min(T_, q0 + 64), a.q_block, Dh, tid);
      tv.load_div(rbase, r_sn, q0 + 64, min(T_, q0 + kWideRows), a.q_block, Dh, tid);
    }
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int ka = c0 + 32 * sb;
      const int cls = block_class(q0 + qw, ka, W);  // uniform over the wave
      if (cls == 0) continue;
      f32x16 s = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) s = mma32(frag_rows<KP>(sk, 32 * sb, 16 * ks), qf[ks], s);  // S^T[key][query]
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = s[i];
      if (cls == 2) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int j = ka + 8 * (i >> 2) + 4 * h + (i & 3);
          x[i] = ((j >= lo) & (j <= hi)) ? x[i] : kNegInf;
        }
      }
      float smax = x[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) smax = fmaxf(smax, x[i]);
      smax = fmaxf(smax, __shfl_xor(smax, 32));  // the two halves of the wave hold the same queries
      const float mloc = smax * a.scale_log2;    // scale_log2 > 0
      // The softmax reference m_run moves only when a block's maximum exceeds it by more than 8 (log2
      // units): exponents then stay <= 8, and the rescale of O and l (and its exp) is skipped in most steps.
      // O and l share the reference, so O / l and lse are unchanged.
      if (__builtin_amdgcn_ballot_w64(mloc > m_run + 8.f)) {  // uniform
        const float m_new = fmaxf(m_run, mloc);
        const float alpha = m_new == kNegInf ? 1.f : fast_exp2(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) o[db] *= alpha;
        m_run = m_new;
      }
      const float mu = m_run == kNegInf ? 0.f : m_run;  // every score of this lane is masked while -inf
      float pv[16], ps = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        pv[i] = fast_exp2(x[i] * a.scale_log2 - mu);
        ps += pv[i];
      }
      l_run += ps;
      const bf16x8 p0 = pack8(pv, 0), p1 = pack8(pv, 1);
#pragma unroll
      for (int db = 0; db < DB; ++db) {  // O^T = V^T P^T, keys in accumulator-row order
        o[db] = mma32(frag_cols<KP>(sv, 32 * sb, 32 * db), p0, o[db]);
        o[db] = mma32(frag_cols<KP>(sv, 32 * sb + 16, 32 * db), p1, o[db]);
      }
    }
  }

  // ---- epilogue: normalise, gate, mix.  Lane (c32, h) holds dims 32 db + 8 j + 4 h .. +3 of its query ----
  if (nch == 0) {  // no key chunk: the remote rows load here
    tk.load_div(rbase, r_sn, q0, min(T_, q0 + 64), a.q_block, Dh, tid);
    tv.load_div(rbase, r_sn, q0 + 64, min(T_, q0 + kWideRows), a.q_block, Dh, tid);
  }
  lds_barrier();  // every wave is done with the key / value buffers
  tk.template store<KP>(SQ, tid);
  tv.template store<KP>(SQ + TILE, tid);
  lds_barrier();
  const float l = l_run + __shfl_xor(l_run, 32);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  float sl = 0.f, sr = 0.f;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * db + 8 * j + 4 * h;
      float rv[4];
      unpack_bf16x4(*reinterpret_cast<const uint2*>(SQ + myrow * KP + d), rv);
      const float4 g4 = *reinterpret_cast<const float4*>(gls + d);
      const float4 r4 = *reinterpret_cast<const float4*>(grs + d);
#pragma unroll
      for (int c = 0; c < 4; ++c) o[db][4 * j + c] = round_t<T>(o[db][4 * j + c] * inv);
      sl += o[db][4 * j] * g4.x + o[db][4 * j + 1] * g4.y + o[db][4 * j + 2] * g4.z + o[db][4 * j + 3] * g4.w;
      sr += rv[0] * r4.x + rv[1] * r4.y + rv[2] * r4.z + rv[3] * r4.w;
    }
  sl += __shfl_xor(sl, 32);
  sr += __shfl_xor(sr, 32);
  const float mm = fmaxf(sl, sr);
  const float el = __expf(sl - mm), er = __expf(sr - mm);
  const float wl = el / (el + er), wr = er / (el + er);
  // y rows [0, 128) in place of the remote rows: lane (c32, h) is the only reader and writer of its dims
  T* SY = SQ;
  T* SO = SKV + 2 * TILE;  // o_local rows [0, 128)
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * db + 8 * j + 4 * h;
      float rv[4], yv[4];
      unpack_bf16x4(*reinterpret_cast<const uint2*>(SQ + myrow * KP + d), rv);
#pragma unroll
      for (int c = 0; c < 4; ++c) yv[c] = wl * o[db][4 * j + c] + wr * rv[c];
      *reinterpret_cast<uint2*>(SY + myrow * KP + d) = make_uint2(pack_bf16x2(yv[0], yv[1]), pack_bf16x2(yv[2], yv[3]));
      *reinterpret_cast<uint2*>(SO + myrow * KP + d) =
          make_uint2(pack_bf16x2(o[db][4 * j], o[db][4 * j + 1]), pack_bf16x2(o[db][4 * j + 2], o[db][4 * j + 3]));
    }
  // o_local, lse and w feed only the backward: a forward-only call passes null for them
  if (qi < T_ && h == 0) {
    const int64_t idx = ((int64_t)b * a.H + hd) * T_ + qi;
    if (a.lse) a.lse[idx] = l > 0.f ? (m_run + __log2f(l)) * kLn2 : kNegInf;
    if (a.w) a.w[idx] = wl;
  }
  lds_barrier();
  T* ybase = static_cast<T*>(a.y) + b * a.y_sb + hd * a.y_sh;
  store_tile<T, DHP, KP>(ybase, a.y_st, SY, q0, T_, Dh);
  store_tile<T, DHP, KP>(ybase, a.y_st, SY + TILE, q0 + 64, T_, Dh);
  if (a.ol) {
    T* obase = static_cast<T*>(a.ol) + b * a.o_sb + hd * a.o_sh;
    store_tile<T, DHP, KP>(obase, a.o_st, SO, q0, T_, Dh);
    store_tile<T, DHP, KP>(obase, a.o_st, SO + TILE, q0 + 64, T_, Dh);
  }
}

}  // namespace

bool wide_bwd(const LocalArgs& a, int dtype, int dhp) {
  return dtype == LLATTN_BF16 && dhp <= 128 && a.W > 64 && strides_fit_32bit(a);
}

bool fwd32(const LocalArgs& a, int dtype, int dhp) {
  return dtype == LLATTN_BF16 && dhp <= 128 && strides_fit_32bit(a);
}

void launch_fwd32(const LocalArgs& a, int dhp, hipStream_t stream) {
  const int n = a.B * a.H * ((a.T + kWideRows - 1) / kWideRows);
  switch (dhp) {
    case 32: hipLaunchKernelGGL(local_fwd32_kernel<32>, dim3(n), dim3(256), 0, stream, a); break;
    case 64: hipLaunchKernelGGL(local_fwd32_kernel<64>, dim3(n), dim3(256), 0, stream, a); break;
    case 96: hipLaunchKernelGGL(local_fwd32_kernel<96>, dim3(n), dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL(local_fwd32_kernel<128>, dim3(n), dim3(256), 0, stream, a); break;
  }
}

int wide_gate_rows(const LocalArgs& a) { return a.B * ((a.T + kWideRows - 1) / kWideRows); }

template <int DHP>
void launch_wide(const LocalArgs& a, int n, hipStream_t stream) {
  hipLaunchKernelGGL(local_bwd_wq_kernel<DHP>, dim3(n), dim3(256), 0, stream, a);
  hipLaunchKernelGGL(local_bwd_wkv_kernel<DHP>, dim3(n), dim3(256), 0, stream, a);
}

void launch_bwd_wide(const LocalArgs& a, int dhp, hipStream_t stream) {
  const int n = a.B * a.H * ((a.T + kWideRows - 1) / kWideRows);
  switch (dhp) {
    case 32: launch_wide<32>(a, n, stream); break;
    case 64: launch_wide<64>(a, n, stream); break;
    case 96: launch_wide<96>(a, n, stream); break;
    default: launch_wide<128>(a, n, stream); break;
  }
}

}  // namespace llattn
