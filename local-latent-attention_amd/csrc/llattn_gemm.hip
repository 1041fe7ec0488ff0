// Projection GEMMs of the local+latent block on bf16 MFMA for gfx950.
//
// C[m][n] = sum_k A(m, k) * B(n, k)  (+ bias[n])  (+ C[m][n] when accumulating)
//
// A and B are bf16 and each is stored either k-contiguous ("A[M][K]",
// "B[N][K]") or m/n-contiguous ("A[K][M]", "B[K][N]"), which covers every
// projection of the block without a transpose copy:
//   forward   y  = x W^T + b      A = x [M][K],   B = W [N][K]
//   input grad dx = dy W          A = dy [M][K],  B = W stored [K][N]
//   weight grad dW = dy^T x       A = dy stored [K][M], B = x stored [K][N]
//
// Tiling: a 256-thread workgroup (4 waves, 2 x 2) owns a 256 x 256 tile of C;
// each wave owns 128 x 128 (64 accumulators of 16 x 16, v_mfma_f32_16x16x32_bf16,
// held in AGPRs).  K advances in steps of 64 through two LDS stages of 64 KB.
// Tiles move from HBM to LDS with buffer_load_dwordx4 ... lds (no register
// staging); a step's loads land while the previous step's 128 MFMAs per wave
// run, and the next sub-step's fragments are read from LDS meanwhile.
//
// LDS layouts (XOR-swizzled at 16-byte granularity, bank-conflict free):
//   k-contiguous tile  [256 rows][64 k]:  chunk c (8 k) of row r at c ^ (r & 7) (A), or at
//                                         c ^ ((r & 3) | (bit 3 of r at bit 2)) (permuted B reads)
//   mn-contiguous tile [64 k][256 cols]:  chunk c (8 cols) of k-row k at c ^ 2(k & 3)
// Operands of one MFMA: lane (r, g) (r = lane % 16, g = lane / 16) supplies
// row r's eight k values 8g .. 8g+7 of a 32-k sub-step -- one ds_read_b128 from a
// k-contiguous tile, two ds_read_b64_tr_b16 from an mn-contiguous one.  Both
// operands use the same k assignment, so the contraction is exact whichever
// layout each comes from.
//
// Split-K (for the weight gradients, whose M x N is small and K = tokens is
// large): split s covers the 64-wide k steps [s*P/S, (s+1)*P/S) of P and writes fp32 partials; an
// ordered reduction adds them (deterministic, no atomics).
//
// Split-head C (llattn_heads_layout, the q|k|v projection output stored as per-sequence head slabs): the
// persistent kernel's stores take each 8-column piece to its slab; the arithmetic is the same.
//
// K need not be a multiple of the step: the last steps read zero past K.  Rows of an m/n-contiguous
// operand past K lie beyond its buffer extent and read zero by themselves; a k-contiguous operand
// (K a multiple of 8) masks the lanes whose 8 k values start at or past K with an out-of-range
// offset (kmask), so no lane reads the next row's elements.
#include <type_traits>

#include "llattn_abi.h"
#include "llattn_device.h"
#include "llattn_heads.h"

namespace llattn {
namespace gemm {

constexpr int BM = 256, BN = 256;  // output tile

enum Epi { EPI_BF16 = 0, EPI_F32 = 1, EPI_PART = 2 };

struct GemmArgs {
  int M, N, K, k_pairs, n_split, tiles_m, tiles_n, accumulate;  // k_pairs: 64-wide k steps, ceil(K / 64)
  const uint16_t* A; int64_t lda, a_bytes;
  const uint16_t* B; int64_t ldb, b_bytes;
  void* C; int64_t ldc;
  const float* bias;
  float* part;     // split-K partials [S][M][N], then (rowsum) [S][M]
  float* rowsum;   // fp32 [M] or null: sum_k A(m, k), from a column of ones in place of B's column N
  // bf16 C only: C[m][n] += ra[(m / T) * n_seg + (m % T) / seg][n] / divisor for each of up to two addends
  const uint16_t* ra_ptr[2];
  int64_t ra_ld[2];
  int ra_T[2], ra_seg[2], ra_nseg[2], ra_div[2];
  // bf16 C only: LLATTN_ACT_GELU writes C = gelu(pre), aux = gelu'(pre); LLATTN_ACT_MUL_AUX scales C by aux
  int act;
  uint16_t* aux;
  int64_t ld_aux;
  HeadsMap ch;  // bf16 C stored split-head (ch.T > 0; persistent kernel)
};

// Exact GELU u * Phi(u) of the reference FeedForward (reference models.py:57, F.gelu) and its derivative
// Phi(u) + u phi(u), in fp32.  erf comes from Abramowitz & Stegun 7.1.26 (Handbook of Mathematical
// Functions): erf(z) = 1 - t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-z^2), t = 1 / (1 + p z), z >= 0,
// absolute error below 1.5e-7 (far under the bf16 rounding of the outputs).  With z = |u| / sqrt(2),
// exp(-z^2) = exp(-u^2 / 2) is also the Gaussian density's exponential, so Phi and phi share one exp:
//   q = t P(t) exp(-u^2/2) / 2,  Phi(u) = 1 - q (u >= 0) or q (u < 0),  phi(u) = exp(-u^2/2) / sqrt(2 pi).
struct NormalCdf {
  float cdf, pdf;
};
__device__ __forceinline__ NormalCdf normal_cdf_pdf(float u) {
  constexpr float p = 0.3275911f, a1 = 0.254829592f, a2 = -0.284496736f, a3 = 1.421413741f,
                  a4 = -1.453152027f, a5 = 1.061405429f;
  const float z = fabsf(u) * 0.70710678118654752f;
  const float t = __builtin_amdgcn_rcpf(fmaf(p, z, 1.f));
  const float poly = t * fmaf(t, fmaf(t, fmaf(t, fmaf(t, a5, a4), a3), a2), a1);
  const float e = __builtin_amdgcn_exp2f(-0.5f * 1.4426950408889634f * u * u);  // exp(-u^2 / 2)
  const float q = 0.5f * poly * e;
  return NormalCdf{u >= 0.f ? 1.f - q : q, e * 0.39894228040143268f};
}
// gelu(u) and gelu'(u) of one value
__device__ __forceinline__ void gelu_pair(float u, float& g, float& gp) {
  const NormalCdf n = normal_cdf_pdf(u);
  g = u * n.cdf;
  gp = fmaf(u, n.pdf, n.cdf);
}
// Eight bf16 pre-activations (packed pairs; the activation acts on the bf16-rounded value, as bf16
// autocast does) -> gelu and gelu' as bf16.
__device__ __forceinline__ void gelu_bf16x8(uint4 x, uint4& g, uint4& gp) {
  const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
  uint32_t o[4], d[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float g0, g1, p0, p1;
    gelu_pair(__uint_as_float(xs[e] << 16), g0, p0);
    gelu_pair(__uint_as_float(xs[e] & 0xffff0000u), g1, p1);
    o[e] = pack_bf16x2(g0, g1);
    d[e] = pack_bf16x2(p0, p1);
  }
  g = make_uint4(o[0], o[1], o[2], o[3]);
  gp = make_uint4(d[0], d[1], d[2], d[3]);
}
// bf16 x * s elementwise (eight packed values each)
__device__ __forceinline__ uint4 mul_bf16x8(uint4 x, uint4 s) {
  const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ss[4] = {s.x, s.y, s.z, s.w};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = pack_bf16x2(__uint_as_float(xs[e] << 16) * __uint_as_float(ss[e] << 16),
                       __uint_as_float(xs[e] & 0xffff0000u) * __uint_as_float(ss[e] & 0xffff0000u));
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// Row of addend q (0, 1) that C row m reads, and its scale (the pooled gradient broadcast to its tokens).
__device__ __forceinline__ const uint16_t* rowadd_row(const GemmArgs& a, int q, int m, float& sc) {
  const int T = a.ra_T[q], t = m % T, s = t / a.ra_seg[q];
  sc = a.ra_div[q] == LLATTN_DIV_COUNT ? 1.f / (float)(min((s + 1) * a.ra_seg[q], T) - s * a.ra_seg[q])
     : a.ra_div[q] == LLATTN_DIV_SEG ? 1.f / (float)a.ra_seg[q] : 1.f;
  return a.ra_ptr[q] + ((int64_t)(m / T) * a.ra_nseg[q] + s) * a.ra_ld[q];
}
__device__ __forceinline__ void add_bf16x4(uint2 u, float sc, float (&v)[4]) {
  v[0] += sc * __uint_as_float(u.x << 16);
  v[1] += sc * __uint_as_float(u.x & 0xffff0000u);
  v[2] += sc * __uint_as_float(u.y << 16);
  v[3] += sc * __uint_as_float(u.y & 0xffff0000u);
}
__device__ __forceinline__ void rowadd4(const GemmArgs& a, int q, int m, int c, float (&v)[4]) {
  float sc;
  const uint16_t* p = rowadd_row(a, q, m, sc);
  add_bf16x4(*reinterpret_cast<const uint2*>(p + c), sc, v);
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void gbl_void;
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

typedef int i32x4 __attribute__((ext_vector_type(4)));

// LDS byte address of a pointer into shared memory
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, gfx9 family

// One wave copies 64 x 16 bytes from global memory into the 1 KB LDS block at
// `dst` (lane i lands at dst + 16 i) with buffer_load_dwordx4 ... lds: the
// step's base address lives in the scalar buffer descriptor and each lane
// adds its fixed 32-bit offset.  Offsets past the descriptor's extent read 0.
// Written as inline asm so that the compiler does not see an LDS write in
// flight: it would otherwise make every later LDS read wait for all of it
// (vmcnt(0)), although the reads target another stage.  The main loop waits
// for these loads itself (vmcnt) before the barrier that publishes them.
// The descriptor and the LDS address are wave-uniform at every call; readfirstlane states it for the
// cases where the compiler cannot prove it (it then keeps them in SGPRs, as the instruction requires).
__device__ __forceinline__ void dma_block(const i32x4& rs, uint32_t off, const unsigned char* dst) {
  const i32x4 srs = {__builtin_amdgcn_readfirstlane(rs[0]), __builtin_amdgcn_readfirstlane(rs[1]),
                     __builtin_amdgcn_readfirstlane(rs[2]), __builtin_amdgcn_readfirstlane(rs[3])};
  const uint32_t sdst = __builtin_amdgcn_readfirstlane(lds_addr(dst));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(off), "s"(srs), "s"(sdst)
               : "memory", "m0");
}

// s_waitcnt immediates (gfx9 encoding: vmcnt [3:0]+[15:14], expcnt [6:4], lgkmcnt [11:8]);
// issued through the builtin so that the compiler's own wait insertion sees them.
constexpr int wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0070 | 0x0F00; }       // vmcnt(n)
constexpr int wait_vm_lgkm0(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0070; }        // vmcnt(n) lgkmcnt(0)

// An offset past every operand extent (operands are below 4 GiB - 16 bytes): the lane reads zero.
constexpr uint32_t kOffPastK = 0xFFFFFFF0u;
// A k-contiguous lane's offset for a step whose K tail starts `klim` elements in, its chunk starting at kc.
__device__ __forceinline__ uint32_t kmask(uint32_t off, int kc, int klim) { return kc < klim ? off : kOffPastK; }

// Buffer descriptor of an operand from step k0 on (`bytes`: storage extent of the operand).
template <bool KMAJ>
__device__ __forceinline__ i32x4 step_rsrc(const uint16_t* base, int64_t ld, int64_t bytes, int k0) {
  const int64_t skip = (KMAJ ? (int64_t)k0 : (int64_t)k0 * ld) * 2;
  const uint64_t addr = reinterpret_cast<uint64_t>(base) + (uint64_t)skip;
  // a step wholly past K can start beyond a small operand's end: extent 0, every lane reads zero
  const int64_t ext = bytes > skip ? bytes - skip : 0;
  return i32x4{(int)(uint32_t)addr, (int)((addr >> 32) & 0xffff), (int)(uint32_t)ext, kRsrcWord3};
}

// 64-k LDS stages (two of 64 KB), shared by gemm_kernel and the persistent kernel.  k-contiguous tiles:
// 256 rows of 128 bytes, 16-byte chunk c of row r at slot c ^ pswz(r) (A fragments read rows o16 + r, eight
// consecutive rows per LDS cycle -> r & 7; permuted B fragments read rows o16 + 8 (r / 4) + r % 4 ->
// (r & 3) | (bit 3 of the row at bit 2); both conflict-free).  mn-contiguous tiles: 64 k-rows of 512 bytes,
// chunk c of k-row k at c ^ 2 (k & 3) (transposing reads, conflict-free).
constexpr int PBK = 64;                  // k per LDS stage
constexpr int PTILE = BM * PBK * 2;      // 32 KB per operand per stage
constexpr int PSTAGE = 2 * PTILE;        // A then B
constexpr int PDMA = PTILE / 1024 / 4;   // 1 KB DMA blocks per wave per operand and step (8)

template <bool PERM>
__device__ __forceinline__ int pswz(int row) {
  return PERM ? ((row & 3) | (((row >> 3) & 1) << 2)) : (row & 7);
}

// Byte offsets (relative to the operand base at the step's first k) of this lane's 16-byte chunk in each
// of the wave's 8 DMA blocks of a 64-k operand tile (rows / columns [o0, o0 + 256)).  k-contiguous: block i
// = rows 8 (8 wave + i) .. + 7, lane -> row + lane / 8, LDS slot lane % 8 receives the row's chunk
// (lane % 8) ^ pswz(row); rows past omax are clamped to a valid row (their outputs are never stored).
// mn-contiguous: block i = k-rows 2 (8 wave + i) + lane / 32, 32 chunks each; columns clamped likewise.
// kc: first k of the lane's chunk (k-contiguous K tail; mn-contiguous rows past K lie beyond the extent).
template <bool KMAJ, bool PERM = false>
__device__ __forceinline__ void tile_offsets64(uint32_t (&off)[PDMA], int (&kc)[PDMA], int64_t ld, int o0, int omax,
                                               int wave, int lane) {
#pragma unroll
  for (int i = 0; i < PDMA; ++i) {
    const int bi = wave * PDMA + i;
    if constexpr (KMAJ) {
      const int row = 8 * bi + (lane >> 3);
      const int c = (lane & 7) ^ pswz<PERM>(row);
      off[i] = (uint32_t)(((int64_t)min(o0 + row, omax - 1) * ld + 8 * c) * 2);
      kc[i] = 8 * c;
    } else {
      const int k = 2 * bi + (lane >> 5);
      const int c = (lane & 31) ^ (2 * (k & 3));
      off[i] = (uint32_t)(((int64_t)k * ld + min(o0 + 8 * c, omax - 8)) * 2);
      kc[i] = 0;
    }
  }
}

// 8 k values (32h + 8g .. + 7 of a 64-k stage) of tile row / column o16 + r for lane (r, g).  PERM
// (k-contiguous B only): lane r reads row o16 + 8 (r / 4) + r % 4 instead, so that with o16 = 32p + 4u the
// output columns a lane accumulates for the block pair (u = 0, 1) are 8 consecutive ones.
template <bool KMAJ, bool PERM = false>
__device__ __forceinline__ bf16x8 frag64(const unsigned char* tile, int o16, int r, int g, int h) {
  if constexpr (KMAJ) {
    const int row = PERM ? o16 + 8 * (r >> 2) + (r & 3) : o16 + r;
    return *reinterpret_cast<const bf16x8*>(tile + row * 128 + (((4 * h + g) ^ pswz<PERM>(row)) << 4));
  } else {
    // transposing reads: the 16 lanes of group g supply k-rows kb + j/4, 8 bytes at column o16 + 4(j%4);
    // lane r receives column o16 + r of those four rows
    const int kb = 32 * h + 8 * g;
    const int col = o16 + 4 * (r & 3), chunk = col >> 3, inner = (col & 7) << 1;
    bf16x4 hv[2];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int k = kb + 4 * half + (r >> 2);
      const unsigned char* p = tile + k * 512 + ((chunk ^ (2 * (k & 3))) << 4) + inner;
      hv[half] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4*)(p));
    }
    return bf16x8{hv[0][0], hv[0][1], hv[0][2], hv[0][3], hv[1][0], hv[1][1], hv[1][2], hv[1][3]};
  }
}

// RS: row sums of A for an N with no spare column (a multiple of 256): every lane adds the 8 k values of each of
// its A fragments into one fp32 sum per fragment block (v_dot2 against a pair of ones, 32 per 32-k sub-step,
// beside the 64 products), and the waves that own the left half of the first tile column store them.
//
// Pipeline (as the persistent kernel's, one tile per workgroup): step kt (64 k) lives in stage kt % 2;
//   sub-step 0: 64 MFMAs on k 0..31, with the fragment reads of k 32..63;
//   wait for this wave's DMA of step kt + 1 (the youngest load: vmcnt(0)) and its reads; barrier;
//   sub-step 1: 64 MFMAs on k 32..63, with the fragment reads of step kt + 1's k 0..31 and the DMA of step
//               kt + 2 into this step's stage (past the last step: the last step again, never read).
// No stores are in flight before the epilogue, so the waits are exact.
template <bool AK, bool BKM, int EPI, bool RS = false>
__global__ __launch_bounds__(256) void gemm_kernel(const GemmArgs a) {
  // bf16 output from a k-contiguous B: permuted B fragments, so each lane writes 16-byte rows directly
  constexpr bool PB = BKM && EPI == EPI_BF16;
  __shared__ __align__(1024) unsigned char smem[2 * PSTAGE];
  const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // workgroup -> (split, tile): contiguous ranges per XCD, then groups of 8 tile rows
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int tiles = a.tiles_m * a.tiles_n;
  const int split = bid / tiles, t = bid % tiles;
  constexpr int GM = 8;
  const int group = t / (GM * a.tiles_n), first_m = group * GM;
  const int gm = min(a.tiles_m - first_m, GM);
  const int tm = first_m + (t % (GM * a.tiles_n)) % gm;
  const int tn = (t % (GM * a.tiles_n)) / gm;
  const int m0 = tm * BM, n0 = tn * BN;
  // split s takes 64-wide steps [s P / S, (s+1) P / S): uneven by at most one step
  const int p0 = split * a.k_pairs / a.n_split, p1 = (split + 1) * a.k_pairs / a.n_split;
  const int kbeg = p0 * PBK, nk = p1 - p0;

  f32x4 acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // first B row / column of fragment block j (PB: block pairs interleave in groups of four)
  auto bcol = [&](int j) { return PB ? wn * 128 + 32 * (j >> 1) + 4 * (j & 1) : wn * 128 + 16 * j; };
  uint32_t offa[PDMA], offb[PDMA];
  int kca[PDMA], kcb[PDMA];
  tile_offsets64<AK>(offa, kca, a.lda, m0, a.M, wave, lane);
  tile_offsets64<BKM, PB>(offb, kcb, a.ldb, n0, a.N, wave, lane);
  // Row sums of A: column N of the product (never stored as C) contracts against ones.  It lies in
  // B fragment block `jones` (wave-uniform; -1: not in this wave's columns) at lane r == rones.
  // Only the waves whose columns hold N run the main loop with the substitution (a wave-uniform branch
  // around the whole loop): in the others no select waits for a fragment read in the sub-step that
  // issues it.
  const int nrel = a.N - n0 - wn * 128;
  const int jones = __builtin_amdgcn_readfirstlane((!PB && a.rowsum && nrel >= 0 && nrel < 128) ? (nrel >> 4) : -1);
  const bool lane_ones = (r == (nrel & 15));
  auto ones_fix = [&](bf16x8& f, int j) {
    if (j == jones && lane_ones) {
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (__bf16)1.0f;
    }
  };
  const bool rs_wave = RS && tn == 0 && wn == 0;  // wave-uniform
  float rsum[8];  // RS: lane (r, g)'s part (k = 8g .. 8g+7 of each sub-step) of sum_k A(m0 + wm*128 + 16i + r, k)
#pragma unroll
  for (int i = 0; i < 8; ++i) rsum[i] = 0.f;
  // DMA of this wave's block q (0..7: operand A, 8..15: operand B) of a step into `stage`; klim = K - k0 of
  // the step (wave-uniform): below PBK, k-contiguous lanes whose chunk starts at or past K read zero
  auto dma = [&](const i32x4& rsa, const i32x4& rsb, int stage, int q, int klim) {
    unsigned char* st = smem + stage * PSTAGE;
    if (q < PDMA) {
      const uint32_t o = (AK && klim < PBK) ? kmask(offa[q], kca[q], klim) : offa[q];
      dma_block(rsa, o, st + (wave * PDMA + q) * 1024);
    } else {
      const int qb = q - PDMA;
      const uint32_t o = (BKM && klim < PBK) ? kmask(offb[qb], kcb[qb], klim) : offb[qb];
      dma_block(rsb, o, st + PTILE + (wave * PDMA + qb) * 1024);
    }
  };
  auto step_rsrcs = [&](int kt, i32x4& rsa, i32x4& rsb) {
    const int k0 = kbeg + kt * PBK;
    rsa = step_rsrc<AK>(a.A, a.lda, a.a_bytes, k0);
    rsb = step_rsrc<BKM>(a.B, a.ldb, a.b_bytes, k0);
  };
  auto frag_a = [&](int stage, int h, int i) { return frag64<AK>(smem + stage * PSTAGE, wm * 128 + 16 * i, r, g, h); };
  auto frag_b = [&](auto ones, int stage, int h, int j) {
    bf16x8 f = frag64<BKM, PB>(smem + stage * PSTAGE + PTILE, bcol(j), r, g, h);
    if constexpr (decltype(ones)::value) ones_fix(f, j);
    return f;
  };
  // 64 MFMAs of a sub-step on (ca, cb), the row sums of ca (RS), and per q the reads / DMA `io(q)`
  auto sub = [&](const bf16x8 (&ca)[8], const bf16x8 (&cb)[8], auto io) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      io(q);
#pragma unroll
      for (int u = 0; u < 4; ++u) {  // B first: lane (r, g) accumulates C[m = r][n = 4g + e]
        const int n = 4 * q + u, i = n >> 3, j = n & 7;
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cb[j], ca[i], acc[i][j], 0, 0, 0);
      }
      if constexpr (RS) {  // fragment block q / 2, pairs 2 (q % 2) and 2 (q % 2) + 1 of its 4 bf16 pairs
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        const bf16x2 one2 = {(__bf16)1.0f, (__bf16)1.0f};
        const bf16x8 f = ca[q >> 1];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int pr = 2 * (q & 1) + e;
          rsum[q >> 1] = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{f[2 * pr], f[2 * pr + 1]}, one2, rsum[q >> 1], false);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

#pragma unroll
  for (int s = 0; s < 2; ++s) {
    i32x4 rsa, rsb;
    const int kd = min(s, nk - 1);
    step_rsrcs(kd, rsa, rsb);
#pragma unroll
    for (int q = 0; q < 2 * PDMA; ++q) dma(rsa, rsb, s, q, a.K - (kbeg + kd * PBK));
  }
  __builtin_amdgcn_s_waitcnt(wait_vm(2 * PDMA));  // loads complete in issue order: step 0 has landed
  __builtin_amdgcn_s_barrier();
  bf16x8 fa0[8], fb0[8], fa1[8], fb1[8];  // k 0..31 and 32..63 of a step
  auto main_loop = [&](auto ones) {
#pragma unroll
    for (int i = 0; i < 8; ++i) fa0[i] = frag_a(0, 0, i);
#pragma unroll
    for (int j = 0; j < 8; ++j) fb0[j] = frag_b(ones, 0, 0, j);
    for (int kt = 0; kt < nk; ++kt) {
      const int s = kt & 1;
      __builtin_amdgcn_sched_barrier(0);
      sub(fa0, fb0, [&](int q) {
        if (q < 8) fa1[q] = frag_a(s, 1, q);
        else fb1[q - 8] = frag_b(ones, s, 1, q - 8);
      });
      __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      i32x4 rsa, rsb;
      const int kd = min(kt + 2, nk - 1), klim = a.K - (kbeg + kd * PBK);
      step_rsrcs(kd, rsa, rsb);
      sub(fa1, fb1, [&](int q) {
        if (q < 8) fa0[q] = frag_a(s ^ 1, 0, q);
        else fb0[q - 8] = frag_b(ones, s ^ 1, 0, q - 8);
        dma(rsa, rsb, s, q, klim);
      });
    }
  };
  if (jones >= 0) main_loop(std::true_type{});
  else main_loop(std::false_type{});
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));  // no DMA may land after the workgroup exits

  // ---- epilogue ----
  // The lane's coordinates again, from the exec mask (mbcnt) rather than held in registers across the main
  // loop: held, the pair was spilled to scratch before the loop and reloaded here.
  {
  const int lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)), r = lane & 15, g = lane >> 4;
  if constexpr (PB) {
    // Lane (r, g) holds C[m0 + wm*128 + 16i + r][n0 + wn*128 + 32p + 8g + e'] for e' = 0..7 in
    // acc[i][2p] (e' < 4) and acc[i][2p+1] (e' >= 4): one 16-byte store per (i, p), 16 rows x 64
    // contiguous bytes per instruction, straight from the accumulators.
    const int rowb = m0 + wm * 128 + r, colb = n0 + wn * 128 + 8 * g;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int col = colb + 32 * p;
      float4 b0 = make_float4(0.f, 0.f, 0.f, 0.f), b1 = b0;
      if (a.bias && col < a.N) {
        b0 = *reinterpret_cast<const float4*>(a.bias + col);
        b1 = *reinterpret_cast<const float4*>(a.bias + col + 4);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = rowb + 16 * i;
        if (row >= a.M || col >= a.N) continue;
        const f32x4 u = acc[i][2 * p], w = acc[i][2 * p + 1];
        float v[8] = {u[0] + b0.x, u[1] + b0.y, u[2] + b0.z, u[3] + b0.w,
                      w[0] + b1.x, w[1] + b1.y, w[2] + b1.z, w[3] + b1.w};
        uint16_t* pc = static_cast<uint16_t*>(a.C) + (int64_t)row * a.ldc + col;
        if (a.accumulate) {
          const uint4 o = ld16(pc);
          const uint32_t os[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[2 * e] += __uint_as_float(os[e] << 16);
            v[2 * e + 1] += __uint_as_float(os[e] & 0xffff0000u);
          }
        }
        const uint4 xo = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                                    pack_bf16x2(v[6], v[7]));
        if (a.act == LLATTN_ACT_GELU) {
          uint4 g, gp;
          gelu_bf16x8(xo, g, gp);
          st16(pc, g);
          st16(a.aux + (int64_t)row * a.ld_aux + col, gp);
        } else {
          st16(pc, xo);
        }
      }
    }
  } else {
  // Lane (r, g) holds C[m0 + wm*128 + 16i + r][n0 + wn*128 + 16j + 4g + e].  The
  // values (+ bias) go through LDS so that global writes are whole 16-byte
  // chunks of contiguous rows: each wave stages its 128 x 128 block in its own
  // 32 KB of LDS (bf16: one pass; fp32: two passes of 64 rows) and writes it back
  // row by row.  Every wave's MFMA operand reads are complete (lgkmcnt above);
  // the barrier makes sure no other wave still reads the stages.
  __builtin_amdgcn_s_barrier();
  unsigned char* stg = smem + wave * 32768;
  const int row0 = m0 + wm * 128, col0 = n0 + wn * 128;
  float4 bias4[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int col = col0 + 16 * j + 4 * g;
    bias4[j] = (EPI != EPI_PART && a.bias && col < a.N) ? *reinterpret_cast<const float4*>(a.bias + col)
                                                        : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if constexpr (EPI == EPI_BF16) {
    // bf16 rows of 256 B; 8-byte unit u of row rl stored at u ^ (rl & 15)
    const bool ra0 = a.ra_ptr[0] != nullptr, ra1 = a.ra_ptr[1] != nullptr;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rl = 16 * i + r;
      // broadcast addends of this row: all eight 4-column pieces loaded before the first is used
      uint2 rv[2][8];
      float rsc[2] = {0.f, 0.f};
      if (ra0 || ra1) {
        const int mrow = min(row0 + rl, a.M - 1);  // rows past M are never stored
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          if (q == 0 ? !ra0 : !ra1) continue;
          const uint16_t* p = rowadd_row(a, q, mrow, rsc[q]);
#pragma unroll
          for (int j = 0; j < 8; ++j)  // columns past N are never stored
            rv[q][j] = *reinterpret_cast<const uint2*>(p + min(col0 + 16 * j + 4 * g, a.N - 4));
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float v[4] = {acc[i][j][0] + bias4[j].x, acc[i][j][1] + bias4[j].y, acc[i][j][2] + bias4[j].z,
                      acc[i][j][3] + bias4[j].w};
        if (ra0) add_bf16x4(rv[0][j], rsc[0], v);
        if (ra1) add_bf16x4(rv[1][j], rsc[1], v);
        uint2 x;
        x.x = static_cast<uint32_t>(f2bf(v[0])) | (static_cast<uint32_t>(f2bf(v[1])) << 16);
        x.y = static_cast<uint32_t>(f2bf(v[2])) | (static_cast<uint32_t>(f2bf(v[3])) << 16);
        *reinterpret_cast<uint2*>(stg + rl * 256 + (((4 * j + g) ^ (rl & 15)) << 3)) = x;
      }
    }
    __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));  // this wave's staging writes are visible to itself
#pragma unroll 4
    for (int it = 0; it < 32; ++it) {  // 4 rows x 16 chunks of 16 B per instruction
      const int idx = it * 64 + lane, rl = idx >> 4, c = idx & 15;
      const int row = row0 + rl, col = col0 + 8 * c;
      // units 2c, 2c+1 sit in one 16-byte slot, swapped when rl is odd
      uint4 x = *reinterpret_cast<const uint4*>(stg + rl * 256 + (((2 * c) ^ (rl & 14)) << 3));
      if (rl & 1) x = make_uint4(x.z, x.w, x.x, x.y);
      if (row < a.M && col < a.N) {
        uint16_t* p = static_cast<uint16_t*>(a.C) + (int64_t)row * a.ldc + col;
        if (a.accumulate) {
          const uint4 o = ld16(p);
          const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, os[4] = {o.x, o.y, o.z, o.w};
          uint32_t rs[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float lo = __uint_as_float(xs[e] << 16) + __uint_as_float(os[e] << 16);
            const float hi = __uint_as_float(xs[e] & 0xffff0000u) + __uint_as_float(os[e] & 0xffff0000u);
            rs[e] = static_cast<uint32_t>(f2bf(lo)) | (static_cast<uint32_t>(f2bf(hi)) << 16);
          }
          x = make_uint4(rs[0], rs[1], rs[2], rs[3]);
        }
        uint16_t* pa = a.aux + (int64_t)row * a.ld_aux + col;
        if (a.act == LLATTN_ACT_MUL_AUX) x = mul_bf16x8(x, ld16(pa));
        if (a.act == LLATTN_ACT_GELU) {
          uint4 g, gp;
          gelu_bf16x8(x, g, gp);
          st16(p, g);
          st16(pa, gp);
        } else {
          st16(p, x);
        }
      }
    }
  } else {
    // fp32 rows of 512 B in two passes of 64 rows; 16-byte chunk c of row rl at c ^ (rl & 7)
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      if (pass) __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));  // first pass's readback is done
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int i = 4 * pass + ii, rl = 16 * ii + r;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float4 v = make_float4(acc[i][j][0] + bias4[j].x, acc[i][j][1] + bias4[j].y,
                                       acc[i][j][2] + bias4[j].z, acc[i][j][3] + bias4[j].w);
          *reinterpret_cast<float4*>(stg + rl * 512 + (((4 * j + g) ^ (rl & 7)) << 4)) = v;
        }
      }
      __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));
#pragma unroll 4
      for (int it = 0; it < 32; ++it) {  // 2 rows x 32 chunks per instruction
        const int idx = it * 64 + lane, rl = idx >> 5, c = idx & 31;
        const int row = row0 + 64 * pass + rl, col = col0 + 4 * c;
        float4 v = *reinterpret_cast<const float4*>(stg + rl * 512 + ((c ^ (rl & 7)) << 4));
        if (row < a.M && col < a.N) {
          float* p = EPI == EPI_PART ? a.part + ((int64_t)split * a.M + row) * a.N + col
                                     : static_cast<float*>(a.C) + (int64_t)row * a.ldc + col;
          if (EPI == EPI_F32 && a.accumulate) {
            const float4 o = *reinterpret_cast<const float4*>(p);
            v.x += o.x; v.y += o.y; v.z += o.z; v.w += o.w;
          }
          *reinterpret_cast<float4*>(p) = v;
        } else if (a.rowsum && row < a.M && col == a.N) {  // the ones column: sum_k A(row, k)
          if (EPI == EPI_PART) a.part[(int64_t)a.n_split * a.M * a.N + (int64_t)split * a.M + row] = v.x;
          else a.rowsum[row] = v.x;
        }
      }
    }
    if (rs_wave) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {  // the four lane groups g hold the row's four 8-wide k slices
        float v = rsum[i];
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        const int row = row0 + 16 * i + r;
        if (g != 0 || row >= a.M) continue;
        if (EPI == EPI_PART) a.part[(int64_t)a.n_split * a.M * a.N + (int64_t)split * a.M + row] = v;
        else a.rowsum[row] = v;
      }
    }
  }
  }
  }
}

// Persistent kernel for bf16 C = A Bᵀ (+ bias) (+ row addends) with k-contiguous A and B and no K split:
// one workgroup per CU walks tiles v = blockIdx.x, + gridDim.x, ...
//
// K advances in 64-wide steps through two LDS stages of 64 KB (A then B, 256 rows of 128 bytes each).
// A DMA instruction moves 8 rows x 128 bytes, so every row of a step arrives as one whole cache line.
// Step g's stage is g % 2; the DMA of step g + 2 goes into it once every wave has read it, which the
// barrier in the middle of step g establishes, so the loads of a step have one step of MFMAs to land:
//   sub-step 0: 64 MFMAs on k 0..31 of the stage, with the fragment reads of k 32..63;
//   wait for this wave's DMA of step g + 1 and its fragment reads; barrier;
//   sub-step 1: 64 MFMAs on k 32..63, with the fragment reads of step g + 1's k 0..31 (other stage)
//               and the 16 DMA instructions of step g + 2 (this stage).
// The DMA runs on across tiles (the last two steps of a tile fetch the first two of the next), and the
// epilogue stores straight from the accumulators, so a tile's output drains to memory while the next tile's
// first MFMAs run.  B fragment block j of a wave reads the tile rows wn 128 + 8 r + j (lane r), so lane
// (r, g) accumulates C[16 i + 4 g + e][8 r + j] in acc[i][j][e]: for each (i, e) the eight blocks j hold 8
// consecutive columns, and one 16-byte store per lane writes 4 rows x 256 bytes (two whole cache lines per
// row; 16 rows x 64 bytes per store took 3-8% longer).  The per-lane DMA
// offsets do not depend on the tile or the step (both lie in the scalar buffer descriptor), so the main
// loop does no per-lane address arithmetic.
//
// Waits never count stores: stores may retire before older loads, so a vmcnt that allowed an epilogue's
// stores in flight could pass with DMA data still missing.  The last step of a tile therefore waits for
// all its DMA (the next tile's steps 0 and 1) before the epilogue issues its stores; the next tile's first
// barrier then waits for nothing in vmcnt, and every later barrier waits for vmcnt(0), the youngest
// load being the DMA it publishes (the stores have had a step to drain by then).
// Buffer descriptor of a k-contiguous operand from row o0 and k0 on.  Rows past the operand read zero
// (their offsets are past `bytes`); they only feed outputs that are never stored.
__device__ __forceinline__ i32x4 tile_rsrc(const uint16_t* base, int64_t ld, int64_t bytes, int o0, int k0) {
  const int64_t skip = ((int64_t)o0 * ld + k0) * 2;
  const uint64_t addr = reinterpret_cast<uint64_t>(base) + (uint64_t)skip;
  const int64_t ext = bytes > skip ? bytes - skip : 0;
  return i32x4{(int)(uint32_t)addr, (int)((addr >> 32) & 0xffff), (int)(uint32_t)ext, kRsrcWord3};
}

// tile v -> origin: contiguous tile ranges per XCD, then groups of 8 tile rows
__device__ __forceinline__ void tile_origin(const GemmArgs& a, int v, int total, int& m0, int& n0) {
  const int t = xcd_remap(v, total);
  constexpr int GM = 8;
  const int group = t / (GM * a.tiles_n), first_m = group * GM;
  const int gm = min(a.tiles_m - first_m, GM);
  // wave-uniform by construction; readfirstlane keeps them in SGPRs (the DMA descriptors need scalars)
  m0 = __builtin_amdgcn_readfirstlane((first_m + (t % (GM * a.tiles_n)) % gm) * BM);
  n0 = __builtin_amdgcn_readfirstlane(((t % (GM * a.tiles_n)) / gm) * BN);
}

// RA: the row addends of GemmArgs (ra_ptr) are added before the rounding, after the bias, in the same order
// as gemm_kernel's bf16 epilogue.
template <int ACT, bool CH = false, bool RA = false>
__global__ __launch_bounds__(256) void gemm_persistent_kernel(const GemmArgs a) {
  __shared__ __align__(1024) unsigned char smem[2 * PSTAGE];
  __shared__ __align__(16) float sbias[2][BN];  // bias of the tile being finished / fetched, by tile parity
  const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int total = a.tiles_m * a.tiles_n, nk = a.k_pairs;  // 64-wide k steps per tile (>= 2: launcher pads K)

  // DMA block i of this wave: rows 8 (8 wave + i) .. + 7 of the operand tile; lane -> row + lane / 8, and
  // its LDS slot lane % 8 receives the row's chunk (lane % 8) ^ pswz(row).  kc*: first k of that chunk.
  uint32_t offa[PDMA], offb[PDMA];
  int kca[PDMA], kcb[PDMA];
#pragma unroll
  for (int i = 0; i < PDMA; ++i) {
    const int row = 8 * (wave * PDMA + i) + (lane >> 3);
    // B: row n of the tile sits at LDS row position n with bits 0 and 3 swapped, its chunk c at slot
    // c ^ ((position >> 4) & 7): the 16 rows 8 r + j (r = 0..15) of fragment block j then alternate
    // between the two halves of the banks and take eight distinct slots in each (conflict-free; with the
    // rows in place all 16 fell in one half)
    const int brow = (row & ~9) | ((row & 1) << 3) | ((row >> 3) & 1);
    const int ca = (lane & 7) ^ pswz<false>(row), cb = (lane & 7) ^ ((row >> 4) & 7);
    offa[i] = (uint32_t)(((int64_t)row * a.lda + 8 * ca) * 2);
    offb[i] = (uint32_t)(((int64_t)brow * a.ldb + 8 * cb) * 2);
    kca[i] = 8 * ca;
    kcb[i] = 8 * cb;
  }
  // LDS byte offsets within a stage of this lane's fragment of sub-step h (k 32h .. 32h + 31); the B row
  // wn 128 + 8 r + j sits at position wn 128 + 16 (r >> 1) + (r & 1) + 8 (j & 1) + (j & 6), swizzle r >> 1
  const int arow = r;
  uint32_t abase[2], bbase[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    abase[h] = arow * 128 + (((4 * h + g) ^ pswz<false>(arow)) << 4);
    bbase[h] = PTILE + (16 * (r >> 1) + (r & 1)) * 128 + (((4 * h + g) ^ (r >> 1)) << 4);
  }
  // fragment block i of A (rows wm*128 + 16i + r), j of B (rows wn*128 + 8r + j)
  auto frag_a = [&](int stage, int h, int i) {
    return *reinterpret_cast<const bf16x8*>(smem + stage * PSTAGE + abase[h] + (wm * 128 + 16 * i) * 128);
  };
  auto frag_b = [&](int stage, int h, int j) {
    return *reinterpret_cast<const bf16x8*>(smem + stage * PSTAGE + bbase[h] +
                                            (wn * 128 + 8 * (j & 1) + (j & 6)) * 128);
  };
  // DMA block q (0..7: A, 8..15: B) of a step into `stage`; klim = K - k0 of the step (K tail: a lane whose
  // chunk starts at or past K reads zero)
  auto dma = [&](const i32x4& rsa, const i32x4& rsb, int stage, int q, int klim) {
    unsigned char* st = smem + stage * PSTAGE;
    if (q < PDMA) {
      const uint32_t o = klim < PBK ? kmask(offa[q], kca[q], klim) : offa[q];
      dma_block(rsa, o, st + (wave * PDMA + q) * 1024);
    } else {
      const int qb = q - PDMA;
      const uint32_t o = klim < PBK ? kmask(offb[qb], kcb[qb], klim) : offb[qb];
      dma_block(rsb, o, st + PTILE + (wave * PDMA + qb) * 1024);
    }
  };

  // C through a range-checked buffer (a masked lane's offset is past the extent; split-head C: the whole matrix)
  const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.C, (CH ? (int64_t)a.M * a.ldc : (int64_t)(a.M - 1) * a.ldc + a.N) * 2);
  const __amdgpu_buffer_rsrc_t raux = make_rsrc(ACT == LLATTN_ACT_GELU ? a.aux : a.C,
                                                ((int64_t)(a.M - 1) * (ACT == LLATTN_ACT_GELU ? a.ld_aux : a.ldc) + a.N) * 2);
  // this wave's 64-column slice of a tile's bias into sbias[slot] (lanes 0..15, 16 bytes each;
  // columns past N, or no bias: zero)
  auto bias_dma = [&](int n0t, int slot) {
    const uint64_t addr = reinterpret_cast<uint64_t>(a.bias) + (uint64_t)n0t * 4;
    const int64_t bytes = a.bias ? (int64_t)(a.N - n0t) * 4 : 0;
    const i32x4 rs{(int)(uint32_t)addr, (int)((addr >> 32) & 0xffff), (int)(uint32_t)bytes, kRsrcWord3};
    if (lane < 16) dma_block(rs, (uint32_t)(wave * 256 + lane * 16), reinterpret_cast<const unsigned char*>(&sbias[slot][wave * 64]));
  };

  int v = blockIdx.x, m0, n0;
  tile_origin(a, v, total, m0, n0);
  // the tile whose steps the DMA fetches after this one, if any
  int vn = v + gridDim.x, m0n = 0, n0n = 0;
  if (vn < total) tile_origin(a, vn, total, m0n, n0n);

  f32x4 acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // prologue: steps 0 and 1 of the first tile and its bias, all landed before the first barrier (as at a
  // tile boundary)
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const i32x4 rsa = tile_rsrc(a.A, a.lda, a.a_bytes, m0, s * PBK), rsb = tile_rsrc(a.B, a.ldb, a.b_bytes, n0, s * PBK);
#pragma unroll
    for (int q = 0; q < 2 * PDMA; ++q) dma(rsa, rsb, s, q, a.K - s * PBK);
  }
  bias_dma(n0, 0);
  __builtin_amdgcn_s_waitcnt(wait_vm(0));
  __builtin_amdgcn_s_barrier();
  bf16x8 fa0[8], fb0[8], fa1[8], fb1[8];  // k 0..31 and 32..63 of a step
#pragma unroll
  for (int i = 0; i < 8; ++i) fa0[i] = frag_a(0, 0, i);
#pragma unroll
  for (int j = 0; j < 8; ++j) fb0[j] = frag_b(0, 0, j);

  int gs = 0;    // global step index of the tile's step 0 (stage of step kt: (gs + kt) % 2)
  int slot = 0;  // sbias slot of the current tile
  // One 64-k step; VMW: the vmcnt wait at its barrier (63: none, step 0 of a tile; 0 otherwise).  The DMA of
  // global step gs+kt+2 fetches the tile's step kt+2, else the next tile's step kt+2-nk, else (last tile)
  // reloads the last step into the free stage, which is never read again.
  auto step = [&](auto vmw_tag, int kt) {
    constexpr int VMW = decltype(vmw_tag)::value;
    const int s = (gs + kt) & 1;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      if (q < 8) fa1[q] = frag_a(s, 1, q);
      else fb1[q - 8] = frag_b(s, 1, q - 8);
#pragma unroll
      for (int u = 0; u < 4; ++u) {  // lane (r, g) accumulates C[m = 4g + e][n = r] of block (i, j)
        const int n = 4 * q + u, i = n >> 3, j = n & 7;
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa0[i], fb0[j], acc[i][j], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(VMW));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const int ka = kt + 2;
    i32x4 rsa, rsb;
    int klim;
    if (ka < nk) {
      rsa = tile_rsrc(a.A, a.lda, a.a_bytes, m0, ka * PBK);
      rsb = tile_rsrc(a.B, a.ldb, a.b_bytes, n0, ka * PBK);
      klim = a.K - ka * PBK;
    } else if (vn < total) {
      rsa = tile_rsrc(a.A, a.lda, a.a_bytes, m0n, (ka - nk) * PBK);
      rsb = tile_rsrc(a.B, a.ldb, a.b_bytes, n0n, (ka - nk) * PBK);
      klim = a.K - (ka - nk) * PBK;
    } else {
      rsa = tile_rsrc(a.A, a.lda, a.a_bytes, m0, (nk - 1) * PBK);
      rsb = tile_rsrc(a.B, a.ldb, a.b_bytes, n0, (nk - 1) * PBK);
      klim = a.K - (nk - 1) * PBK;
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      if (q < 8) fa0[q] = frag_a(s ^ 1, 0, q);
      else fb0[q - 8] = frag_b(s ^ 1, 0, q - 8);
      dma(rsa, rsb, s, q, klim);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int n = 4 * q + u, i = n >> 3, j = n & 7;
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa1[i], fb1[j], acc[i][j], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  while (true) {
    step(std::integral_constant<int, 63>{}, 0);
    for (int kt = 1; kt < nk; ++kt) step(std::integral_constant<int, 0>{}, kt);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(wait_vm(0));  // the next tile's first two steps have landed: no store in flight yet
    bias_dma(vn < total ? n0n : n0, slot ^ 1);  // the next tile's bias, after the DMA of its 2nd step
    // ---- epilogue: lane (r, g) holds C[m0 + wm*128 + 16i + 4g + e][n0 + wn*128 + 8r + j] in acc[i][j][e] ----
    const int rowb = m0 + wm * 128 + 4 * g, col = n0 + wn * 128 + 8 * r;
    float bv[8];  // this lane's 8 bias columns, the same for every row
    {
      const float* bl = &sbias[slot][wn * 128 + 8 * r];
      const float4 b0 = *reinterpret_cast<const float4*>(bl), b1 = *reinterpret_cast<const float4*>(bl + 4);
      bv[0] = b0.x; bv[1] = b0.y; bv[2] = b0.z; bv[3] = b0.w;
      bv[4] = b1.x; bv[5] = b1.y; bv[6] = b1.z; bv[7] = b1.w;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = rowb + 16 * i + e;
        // the accumulators leave the AGPRs here, eight at a time: left to the compiler, all 256 were copied
        // out at the end of the main loop and the register peak pushed the loop's offsets into scratch
        float v8[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v8[j]) : "a"(acc[i][j][e]));
          v8[j] += bv[j];
        }
        if constexpr (RA) {  // addend rows of this output row (rows past M are never stored; rows 8-byte aligned)
          const int m = min(row, a.M - 1), cc = min(col, a.N - 8);  // columns past N are never stored
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            if (!a.ra_ptr[q]) continue;
            const int T = a.ra_T[q], seg = a.ra_seg[q], t = m % T, sg = t / seg;
            const float rsc = a.ra_div[q] == LLATTN_DIV_COUNT ? 1.f / (float)(min((sg + 1) * seg, T) - sg * seg)
                            : a.ra_div[q] == LLATTN_DIV_SEG ? 1.f / (float)seg : 1.f;
            const uint16_t* rap = a.ra_ptr[q] + ((int64_t)(m / T) * a.ra_nseg[q] + sg) * a.ra_ld[q];
            float lo[4] = {v8[0], v8[1], v8[2], v8[3]}, hi[4] = {v8[4], v8[5], v8[6], v8[7]};
            add_bf16x4(*reinterpret_cast<const uint2*>(rap + cc), rsc, lo);
            add_bf16x4(*reinterpret_cast<const uint2*>(rap + cc + 4), rsc, hi);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              v8[u] = lo[u];
              v8[4 + u] = hi[u];
            }
          }
        }
        const uint4 x = make_uint4(pack_bf16x2(v8[0], v8[1]), pack_bf16x2(v8[2], v8[3]),
                                   pack_bf16x2(v8[4], v8[5]), pack_bf16x2(v8[6], v8[7]));
        const uint32_t oc = (row < a.M && col < a.N)
                                ? (CH ? heads_off(a.ch, (uint32_t)row, (uint32_t)col) : (uint32_t)((int64_t)row * a.ldc + col)) * 2u
                                : kOffOOB;
        if constexpr (ACT == LLATTN_ACT_GELU) {
          uint4 gl, gp;
          gelu_bf16x8(x, gl, gp);
          const uint32_t oa = (row < a.M && col < a.N) ? (uint32_t)((int64_t)row * a.ld_aux + col) * 2u : kOffOOB;
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, gl), rc, oc, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, gp), raux, oa, 0, 0);
        } else {
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, x), rc, oc, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (vn >= total) break;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    gs += nk;
    slot ^= 1;
    v = vn;
    m0 = m0n;
    n0 = n0n;
    vn = v + gridDim.x;
    if (vn < total) tile_origin(a, vn, total, m0n, n0n);
  }
  __builtin_amdgcn_s_waitcnt(wait_vm(0));  // no DMA may land after the workgroup exits
}

// C = sum over splits of the partials (+ bias) (+ C), 4 columns per thread.
// Threads past the M x N/4 quads add the row-sum partials [S][M] the same way, one row each.
template <int EPI>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const GemmArgs a, int S) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;  // quad index over M x N/4
  const int nq = a.N / 4;
  const int64_t mn = (int64_t)a.M * a.N;
  if (q >= (int64_t)a.M * nq) {
    const int64_t row = q - (int64_t)a.M * nq;
    if (!a.rowsum || row >= a.M) return;
    const float* p = a.part + (int64_t)S * mn + row;
    float s = p[0];
    for (int i = 1; i < S; ++i) s += p[(int64_t)i * a.M];
    a.rowsum[row] = s;
    return;
  }
  const int row = (int)(q / nq), col = (int)(q % nq) * 4;
  const float* p = a.part + (int64_t)row * a.N + col;
  float4 s = *reinterpret_cast<const float4*>(p);
  int i = 1;
  for (; i + 4 <= S; i += 4) {  // four partials in flight, added in split order
    float4 x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = *reinterpret_cast<const float4*>(p + (i + u) * mn);
#pragma unroll
    for (int u = 0; u < 4; ++u) { s.x += x[u].x; s.y += x[u].y; s.z += x[u].z; s.w += x[u].w; }
  }
  for (; i < S; ++i) {
    const float4 x = *reinterpret_cast<const float4*>(p + i * mn);
    s.x += x.x; s.y += x.y; s.z += x.z; s.w += x.w;
  }
  float v[4] = {s.x, s.y, s.z, s.w};
  if (a.bias) {
    const float4 b4 = *reinterpret_cast<const float4*>(a.bias + col);
    v[0] += b4.x; v[1] += b4.y; v[2] += b4.z; v[3] += b4.w;
  }
  if constexpr (EPI == EPI_F32) {
    float* c = static_cast<float*>(a.C) + (int64_t)row * a.ldc + col;
    if (a.accumulate) {
      const float4 o = *reinterpret_cast<const float4*>(c);
      v[0] += o.x; v[1] += o.y; v[2] += o.z; v[3] += o.w;
    }
    *reinterpret_cast<float4*>(c) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    uint16_t* c = static_cast<uint16_t*>(a.C) + (int64_t)row * a.ldc + col;
    if (a.accumulate) {
      float o[4];
      load4<uint16_t>(c, o);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += o[e];
    }
    if (a.ra_ptr[0]) rowadd4(a, 0, row, col, v);
    if (a.ra_ptr[1]) rowadd4(a, 1, row, col, v);
    if (a.act) {  // the activation acts on the bf16-rounded value
      uint16_t* pa = a.aux + (int64_t)row * a.ld_aux + col;
      float h[4];
      if (a.act == LLATTN_ACT_MUL_AUX) load4<uint16_t>(pa, h);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float xb = round_t<uint16_t>(v[e]);
        if (a.act == LLATTN_ACT_GELU) gelu_pair(xb, v[e], h[e]);
        else v[e] = xb * h[e];
      }
      if (a.act == LLATTN_ACT_GELU) store4<uint16_t>(pa, h);
    }
    store4<uint16_t>(c, v);
  }
}

template <bool AK, bool BKM>
void launch(const GemmArgs& a, int S, int c_dtype, hipStream_t st) {
  const dim3 grid(a.tiles_m * a.tiles_n * S), block(256);
  // row sums with no spare column (N a multiple of 256): the weight-gradient layout only
  const bool rs = !AK && !BKM && a.rowsum && a.N % BN == 0;
  if (S > 1) {
    if (rs) hipLaunchKernelGGL((gemm_kernel<AK, BKM, EPI_PART, !AK && !BKM>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((gemm_kernel<AK, BKM, EPI_PART>), grid, block, 0, st, a);
    const int64_t quads = (int64_t)a.M * (a.N / 4) + (a.rowsum ? a.M : 0);
    const dim3 rg((unsigned)((quads + 255) / 256));
    if (c_dtype == LLATTN_F32)
      hipLaunchKernelGGL((splitk_reduce_kernel<EPI_F32>), rg, block, 0, st, a, S);
    else
      hipLaunchKernelGGL((splitk_reduce_kernel<EPI_BF16>), rg, block, 0, st, a, S);
  } else if (c_dtype == LLATTN_F32) {
    if (rs) hipLaunchKernelGGL((gemm_kernel<AK, BKM, EPI_F32, !AK && !BKM>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((gemm_kernel<AK, BKM, EPI_F32>), grid, block, 0, st, a);
  } else {
    hipLaunchKernelGGL((gemm_kernel<AK, BKM, EPI_BF16>), grid, block, 0, st, a);
  }
}


// ---------------------------------------------------------------------------------------------------------
// Small products: the pooled-latent projection rkv_proj (reference models.py:333-342) and its backward have
// a few hundred rows or a contraction of a few hundred (config 2: 256 x 1024 x 1408 and its transposes).
// On the 256 x 256 tiles they run as ~20 workgroups whose pipelines never fill.  Here: 64 x 64 output tiles,
// one 256-thread workgroup each (4 waves of 32 x 32), the whole contraction per workgroup in 64-wide k
// chunks staged through two LDS panel buffers (the next chunk's loads in flight during the current chunk's
// MFMAs).  Either operand may be k- or m/n-contiguous: k-contiguous rows are copied as 16-byte pieces,
// m/n-contiguous ones are transposed on their way into LDS, so fragments are always k-contiguous.  LDS rows
// of 64 k (128 bytes) with 16-byte chunk c of row r at c ^ ((r >> 1) & 7): conflict-free ds_read_b128.
// ---------------------------------------------------------------------------------------------------------
constexpr int SBT = 64, SBK = 64;

__device__ __forceinline__ int sswz(int row) { return (row >> 1) & 7; }

// This thread's two 16-byte pieces of a 64 x 64 operand panel (rows o0 .., k from k0) -> registers.
template <bool KMAJ>
__device__ __forceinline__ void small_load(uint4 (&v)[2], const uint16_t* base, int64_t ld, int o0, int omax, int k0,
                                           int K, int tid) {
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int q = tid + 256 * u;
    if constexpr (KMAJ) {  // piece: row q / 8, k 8 (q % 8) .. +7
      const int row = o0 + (q >> 3), k = k0 + 8 * (q & 7);
      v[u] = (row < omax && k < K) ? *reinterpret_cast<const uint4*>(base + (int64_t)row * ld + k)
                                   : make_uint4(0u, 0u, 0u, 0u);
    } else {  // piece: k-row q / 8, rows 8 (q % 8) .. +7 of the panel
      const int k = k0 + (q >> 3), row = o0 + 8 * (q & 7);
      v[u] = (k < K && row < omax) ? *reinterpret_cast<const uint4*>(base + (int64_t)k * ld + row)
                                   : make_uint4(0u, 0u, 0u, 0u);
    }
  }
}
template <bool KMAJ>
__device__ __forceinline__ void small_store(const uint4 (&v)[2], unsigned char* panel, int tid) {
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int q = tid + 256 * u;
    if constexpr (KMAJ) {
      const int row = q >> 3, c = q & 7;
      *reinterpret_cast<uint4*>(panel + row * 128 + ((c ^ sswz(row)) << 4)) = v[u];
    } else {  // eight rows of one k: one element each
      const int k = q >> 3, r0 = 8 * (q & 7);
      const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int row = r0 + e;
        *reinterpret_cast<uint16_t*>(panel + row * 128 + (((k >> 3) ^ sswz(row)) << 4) + 2 * (k & 7)) =
            (uint16_t)((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffffu));
      }
    }
  }
}

template <bool AK, bool BKM, int EPI>
__global__ __launch_bounds__(256) void gemm_small_kernel(const GemmArgs a) {
  __shared__ __align__(16) unsigned char As[2][SBT * 128], Bs[2][SBT * 128];
  const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
  const int wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
  const int tn_count = (a.N + SBT - 1) / SBT, tiles = ((a.M + SBT - 1) / SBT) * tn_count;
  // EPI_PART: split blockIdx / tiles takes chunks [s C / S, (s+1) C / S) of the C 64-wide chunks
  const int split = EPI == EPI_PART ? blockIdx.x / tiles : 0, t = EPI == EPI_PART ? blockIdx.x % tiles : blockIdx.x;
  const int tm = t / tn_count, tn = t % tn_count;
  const int m0 = tm * SBT, n0 = tn * SBT;
  const bool want_rowsum = a.rowsum && tn == 0;
  const int call = (a.K + SBK - 1) / SBK;
  const int cbeg = EPI == EPI_PART ? split * call / a.n_split : 0;
  const int nchunks = (EPI == EPI_PART ? (split + 1) * call / a.n_split : call) - cbeg;
  const int kbase = cbeg * SBK;
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float rs = 0.f;  // threads 0..63: the row sum of A row m0 + tid
  // chunk c's loads land in register set c % 4: four chunks in flight ahead of the MFMAs
  uint4 va[4][2], vb[4][2];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if (d < nchunks) {
      small_load<AK>(va[d], a.A, a.lda, m0, a.M, kbase + d * SBK, a.K, tid);
      small_load<BKM>(vb[d], a.B, a.ldb, n0, a.N, kbase + d * SBK, a.K, tid);
    }
  }
  auto chunk = [&](int c, uint4 (&ra)[2], uint4 (&rb)[2]) {
    unsigned char* pa = As[c & 1];
    unsigned char* pb = Bs[c & 1];
    small_store<AK>(ra, pa, tid);
    small_store<BKM>(rb, pb, tid);
    __syncthreads();  // the panels of chunk c are complete; the other buffer (chunk c-1) is no longer read
    if (c + 4 < nchunks) {  // this register set is free again: chunk c + 4
      small_load<AK>(ra, a.A, a.lda, m0, a.M, kbase + (c + 4) * SBK, a.K, tid);
      small_load<BKM>(rb, a.B, a.ldb, n0, a.N, kbase + (c + 4) * SBK, a.K, tid);
    }
    if (want_rowsum && tid < SBT) {
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) {
        const uint4 x = *reinterpret_cast<const uint4*>(pa + tid * 128 + ((cc ^ sswz(tid)) << 4));
        const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) rs += __uint_as_float(w[e] << 16) + __uint_as_float(w[e] & 0xffff0000u);
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // two 32-wide k steps per chunk
      bf16x8 fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = wm * 32 + 16 * i + r, cc = 4 * h + g;
        fa[i] = *reinterpret_cast<const bf16x8*>(pa + row * 128 + ((cc ^ sswz(row)) << 4));
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int row = wn * 32 + 16 * j + r, cc = 4 * h + g;
        fb[j] = *reinterpret_cast<const bf16x8*>(pb + row * 128 + ((cc ^ sswz(row)) << 4));
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
    }
    __syncthreads();  // every wave is done with buffer c & 1 before chunk c + 2 overwrites it
  };
  for (int c = 0; c < nchunks; c += 4) {
    chunk(c, va[0], vb[0]);
    if (c + 1 < nchunks) chunk(c + 1, va[1], vb[1]);
    if (c + 2 < nchunks) chunk(c + 2, va[2], vb[2]);
    if (c + 3 < nchunks) chunk(c + 3, va[3], vb[3]);
  }
  if (want_rowsum && tid < SBT && m0 + tid < a.M) {
    if constexpr (EPI == EPI_PART) a.part[(int64_t)a.n_split * a.M * a.N + (int64_t)split * a.M + m0 + tid] = rs;
    else a.rowsum[m0 + tid] = rs;
  }
  // lane (r, g) holds C[m0 + wm*32 + 16i + r][n0 + wn*32 + 16j + 4g + e]
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = n0 + wn * 32 + 16 * j + 4 * g;
    if (col >= a.N) continue;
    const float4 b4 = (EPI != EPI_PART && a.bias) ? *reinterpret_cast<const float4*>(a.bias + col)
                                                   : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = m0 + wm * 32 + 16 * i + r;
      if (row >= a.M) continue;
      float v[4] = {acc[i][j][0] + b4.x, acc[i][j][1] + b4.y, acc[i][j][2] + b4.z, acc[i][j][3] + b4.w};
      if constexpr (EPI == EPI_PART) {  // this split's fp32 partial [split][M][N]
        *reinterpret_cast<float4*>(a.part + ((int64_t)split * a.M + row) * a.N + col) = make_float4(v[0], v[1], v[2], v[3]);
      } else if constexpr (EPI == EPI_BF16) {
        uint16_t* p = static_cast<uint16_t*>(a.C) + (int64_t)row * a.ldc + col;
        if (a.accumulate) {
          float o[4];
          load4<uint16_t>(p, o);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] += o[e];
        }
        store4<uint16_t>(p, v);
      } else {
        float* p = static_cast<float*>(a.C) + (int64_t)row * a.ldc + col;
        if (a.accumulate) {
          const float4 o = *reinterpret_cast<const float4*>(p);
          v[0] += o.x; v[1] += o.y; v[2] += o.z; v[3] += o.w;
        }
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  }
}

template <bool AK, bool BKM>
void launch_small(const GemmArgs& a, int c_dtype, hipStream_t st) {
  const int tiles = ((a.M + SBT - 1) / SBT) * ((a.N + SBT - 1) / SBT);
  const dim3 block(256);
  if (a.n_split > 1) {  // K splits: fp32 partials, then the ordered reduction of the large products
    hipLaunchKernelGGL((gemm_small_kernel<AK, BKM, EPI_PART>), dim3(tiles * a.n_split), block, 0, st, a);
    const int64_t quads = (int64_t)a.M * (a.N / 4) + (a.rowsum ? a.M : 0);
    const dim3 rg((unsigned)((quads + 255) / 256));
    if (c_dtype == LLATTN_F32) hipLaunchKernelGGL((splitk_reduce_kernel<EPI_F32>), rg, block, 0, st, a, a.n_split);
    else hipLaunchKernelGGL((splitk_reduce_kernel<EPI_BF16>), rg, block, 0, st, a, a.n_split);
    return;
  }
  if (c_dtype == LLATTN_F32) hipLaunchKernelGGL((gemm_small_kernel<AK, BKM, EPI_F32>), dim3(tiles), block, 0, st, a);
  else hipLaunchKernelGGL((gemm_small_kernel<AK, BKM, EPI_BF16>), dim3(tiles), block, 0, st, a);
}

// The small-tile path: no K split requested, no activation or row addends, an output of at most 32 tiles of
// 256 x 256 with one side at most 1024, and a contraction of at most 4096.
bool use_small(const llattn_gemm_desc* d) {
  const int64_t tiles = (int64_t)((d->M + BM - 1) / BM) * ((d->N + BN - 1) / BN);
  return d->split_k == 0 && d->act == LLATTN_ACT_NONE && !d->rowadd[0].ptr && !d->rowadd[1].ptr &&
         d->c_heads.T == 0 && tiles <= 32 &&
         std::min(d->M, d->N) <= 1024 && d->K <= 4096;
}

// K splits of a small product: its 64 x 64 tiles run their chunks one after another, ~0.7 us per 64-wide
// chunk when a few workgroups cover the output, so a long contraction over few tiles is split while the
// splits fit one round on the chip; the ordered reduction then costs ~3.5 us plus its fp32 traffic (E.g.
// the 512 x 64 x 1024 query-block projection of config 4: 8 tiles of 16 chunks, 8 splits of 2.)
int small_split(const llattn_gemm_desc* d) {
  const int64_t tiles = (int64_t)((d->M + SBT - 1) / SBT) * ((d->N + SBT - 1) / SBT);
  const int64_t chunks = (d->K + SBK - 1) / SBK;
  int best = 1;
  double best_t = (double)chunks * 0.7e-6;
  for (int64_t S = 2; S <= std::min<int64_t>(chunks / 2, 16) && tiles * S <= 256; ++S) {
    const double t = (double)((chunks + S - 1) / S) * 0.7e-6 + 3.5e-6 +
                     2.0 * S * d->M * (double)(d->N + (d->a_rowsum ? 1 : 0)) * 4.0 / 5e12;
    if (t < best_t * 0.9) {
      best_t = t;
      best = (int)S;
    }
  }
  return best;
}

// Number of K splits: 1 when the output tiles alone fill most of the chip; otherwise the split count S
// that minimises a time model of the product: the busiest CU runs ceil(tiles S / 256) workgroups of
// 1/S of a tile's k range each (one 128 KB workgroup per CU), plus the fp32 partials that the ordered
// reduction reads and writes (S M N 4 bytes at ~5 TB/s, against a tile rate of ~4.4 TFLOP/s per CU).
// Each split keeps at least four 64-wide k steps.  E.g. 96 tiles (a 4096 x 1408 weight gradient): 8
// splits fill three rounds exactly, where 2 would leave a quarter of the CUs idle.
int resolve_split(const llattn_gemm_desc* d) {
  if (d->split_k > 0) return d->split_k;
  if (d->c_heads.T != 0) return 1;  // a split-head C comes from the persistent kernel
  // so do row addends with a k-contiguous B (an input gradient through the transposed weight)
  if (!d->a_trans && !d->b_trans && (d->rowadd[0].ptr || d->rowadd[1].ptr)) return 1;
  const int64_t tiles = (int64_t)((d->M + BM - 1) / BM) * ((d->N + BN - 1) / BN);
  if (tiles >= 224) return 1;
  const int64_t pairs = (d->K + PBK - 1) / PBK;
  const int64_t smax = std::max<int64_t>(1, pairs / 4);
  const double t_tile = 2.0 * BM * BN * (double)pairs * PBK / 4.4e12;  // seconds per whole tile
  // unsplit, a bf16 product of k-contiguous operands runs on the persistent kernel, whose tiles pay no
  // fill or partial epilogue of their own (config 3's r_out input gradient, 128 tiles of 16 steps with 64
  // valid columns: 25.5 us unsplit against 32.4 us in 2 splits plus their reduction)
  const bool persistent = !d->a_trans && !d->b_trans && d->c_dtype == LLATTN_BF16 && !d->accumulate &&
                          d->act == LLATTN_ACT_NONE;
  int best = 1;
  double best_t = 1e30;
  for (int64_t S = 1; S <= std::min<int64_t>(smax, 64); ++S) {
    // each round of workgroups also pays ~15 us of pipeline fill and partial-tile epilogue, so a split that
    // needs a second round must save more than that (52 tiles, K = 32768: 4 splits in one round 260 us,
    // 9 splits in two rounds ~300 us)
    const double rounds = (double)((tiles * S + 255) / 256);
    const double t = rounds * (t_tile / (double)S + (S == 1 && persistent ? 0.0 : 15e-6)) +
                     (S > 1 ? 2.0 * S * d->M * (double)d->N * 4.0 / 5e12 : 0.0);
    if (t < best_t * 0.999) {
      best_t = t;
      best = (int)S;
    }
  }
  return best;
}

}  // namespace gemm
}  // namespace llattn

using namespace llattn;
using namespace llattn::gemm;

extern "C" size_t llattn_gemm_workspace_size(const llattn_gemm_desc* d) {
  if (!d) return 0;
  const int S = use_small(d) ? small_split(d) : resolve_split(d);
  return S > 1 ? (size_t)S * d->M * (d->N + (d->a_rowsum ? 1 : 0)) * sizeof(float) : 0;
}

extern "C" int32_t llattn_gemm(const llattn_gemm_desc* d, void* workspace, size_t workspace_bytes, void* stream) {
  if (!d) return fail(LLATTN_ERR_SHAPE, "llattn_gemm: null descriptor");
  if (d->M <= 0 || d->N <= 0 || d->K <= 0)
    return fail(LLATTN_ERR_SHAPE, "llattn_gemm: sizes must be positive (M=%d N=%d K=%d)", d->M, d->N, d->K);
  if (d->c_dtype != LLATTN_BF16 && d->c_dtype != LLATTN_F32)
    return fail(LLATTN_ERR_DTYPE, "llattn_gemm: unknown output dtype %d", d->c_dtype);
  const int S = resolve_split(d);
  const int k_pairs = (d->K + PBK - 1) / PBK;
  if ((!d->a_trans || !d->b_trans) && d->K % 8 != 0)
    return fail(LLATTN_ERR_UNSUPPORTED, "llattn_gemm: K=%d must be a multiple of 8 when an operand is k-contiguous",
                d->K);
  if (S < 1 || S > k_pairs)
    return fail(LLATTN_ERR_UNSUPPORTED, "llattn_gemm: %d K splits for K=%d: at most one per %d-wide k step", S, d->K,
                PBK);
  if (d->N % 8 != 0 || (d->a_trans && d->M % 8 != 0))
    return fail(LLATTN_ERR_UNSUPPORTED, "llattn_gemm: N (and M of a transposed A) must be multiples of 8 (M=%d N=%d)",
                d->M, d->N);
  if (!d->A || !d->B || !d->C || !aligned16(d->A) || !aligned16(d->B) || !aligned16(d->C) ||
      (d->bias && !aligned16(d->bias)))
    return fail(LLATTN_ERR_LAYOUT, "llattn_gemm: operands must be non-null and 16-byte aligned");
  if (d->lda % 8 || d->ldb % 8 || d->ldc % 8)
    return fail(LLATTN_ERR_LAYOUT, "llattn_gemm: lda, ldb and ldc must be multiples of 8 elements");
  if (d->lda < (d->a_trans ? d->M : d->K) || d->ldb < (d->b_trans ? d->N : d->K) || d->ldc < d->N)
    return fail(LLATTN_ERR_LAYOUT, "llattn_gemm: leading dimensions smaller than the rows they hold");
  // storage extents of the operands (the last row ends at its used width)
  const int64_t a_bytes = (d->a_trans ? (int64_t)(d->K - 1) * d->lda + d->M : (int64_t)(d->M - 1) * d->lda + d->K) * 2;
  const int64_t b_bytes = (d->b_trans ? (int64_t)(d->K - 1) * d->ldb + d->N : (int64_t)(d->N - 1) * d->ldb + d->K) * 2;
  if (a_bytes > (int64_t)kOffPastK || b_bytes > (int64_t)kOffPastK)
    return fail(LLATTN_ERR_UNSUPPORTED, "llattn_gemm: operands of 4 GiB or more are not supported");
  if (d->a_rowsum && (!d->b_trans || d->c_dtype != LLATTN_F32 || (d->N % BN == 0 && !d->a_trans) ||
                      !aligned16(d->a_rowsum)))
    return fail(LLATTN_ERR_UNSUPPORTED,
                "llattn_gemm: row sums of A need an m/n-contiguous B, fp32 C, an m-contiguous A when N is a multiple "
                "of %d (N=%d) and a 16-byte aligned output", BN, d->N);
  for (int q = 0; q < 2; ++q) {
    const llattn_gemm_rowadd& ra = d->rowadd[q];
    if (!ra.ptr) continue;
    if (d->c_dtype != LLATTN_BF16 || d->a_trans)
      return fail(LLATTN_ERR_UNSUPPORTED, "llattn_gemm: row addends need bf16 C and a k-contiguous A (a_trans = 0)");
    if (ra.rows_per_seq <= 0 || d->M % ra.rows_per_seq || ra.seg <= 0 || ra.n_seg != (ra.rows_per_seq + ra.seg - 1) / ra.seg ||
        (ra.divisor != LLATTN_DIV_COUNT && ra.divisor != LLATTN_DIV_SEG && ra.divisor != LLATTN_DIV_ONE))
      return fail(LLATTN_ERR_SHAPE, "llattn_gemm: row addend %d: M=%d must be whole sequences of %d rows, n_seg=%d "
                  "must be ceil(%d / seg=%d), divisor %d known", q, d->M, ra.rows_per_seq, ra.n_seg, ra.rows_per_seq,
                  ra.seg, ra.divisor);
    if ((uintptr_t)ra.ptr % 8 || ra.ld % 4 || ra.ld < d->N)
      return fail(LLATTN_ERR_LAYOUT, "llattn_gemm: row addend %d must be 8-byte aligned with ld >= N, a multiple of 4", q);
  }
  if (d->act != LLATTN_ACT_NONE) {
    if (d->act != LLATTN_ACT_GELU && d->act != LLATTN_ACT_MUL_AUX)
      return fail(LLATTN_ERR_UNSUPPORTED, "llattn_gemm: unknown activation %d", d->act);
    if (d->c_dtype != LLATTN_BF16 || d->accumulate || d->a_trans || d->rowadd[0].ptr || d->rowadd[1].ptr)
      return fail(LLATTN_ERR_UNSUPPORTED, "llattn_gemm: an activation needs bf16 C, a k-contiguous A, no "
                  "accumulation and no row addends");
    if (!d->aux || !aligned16(d->aux) || d->ld_aux % 8 || d->ld_aux < d->N)
      return fail(LLATTN_ERR_LAYOUT, "llattn_gemm: the activation's aux matrix must be 16-byte aligned with "
                  "ld_aux >= N, a multiple of 8");
    if (((int64_t)(d->M - 1) * d->ld_aux + d->N) * 2 >= (int64_t(1) << 31))
      return fail(LLATTN_ERR_UNSUPPORTED, "llattn_gemm: the activation's aux matrix must be below 2 GiB");
  }
  HeadsMap ch;
  if (const int32_t rc = heads_map("llattn_gemm (C)", &d->c_heads, d->M, d->ldc, d->N, &ch)) return rc;
  if (ch.T && (d->a_trans || d->b_trans || d->c_dtype != LLATTN_BF16 || d->accumulate || d->act != LLATTN_ACT_NONE ||
               d->rowadd[0].ptr || d->rowadd[1].ptr || S != 1))
    return fail(LLATTN_ERR_UNSUPPORTED, "llattn_gemm: a split-head C needs a_trans = b_trans = 0, bf16 C, no "
                "accumulation, activation, row addends or K split");
  const size_t need = llattn_gemm_workspace_size(d);
  if (need && (!workspace || workspace_bytes < need || !aligned16(workspace)))
    return fail(LLATTN_ERR_WORKSPACE, "llattn_gemm: %d K splits need %zu workspace bytes (got %zu)",
                use_small(d) ? small_split(d) : S, need, workspace_bytes);
  GemmArgs a{};
  a.M = d->M; a.N = d->N; a.K = d->K; a.k_pairs = k_pairs; a.n_split = S;
  a.tiles_m = (d->M + BM - 1) / BM; a.tiles_n = (d->N + BN - 1) / BN;
  a.accumulate = d->accumulate;
  a.A = static_cast<const uint16_t*>(d->A); a.lda = d->lda; a.a_bytes = a_bytes;
  a.B = static_cast<const uint16_t*>(d->B); a.ldb = d->ldb; a.b_bytes = b_bytes;
  a.C = d->C; a.ldc = d->ldc;
  a.ch = ch;
  a.bias = d->bias;
  a.part = static_cast<float*>(workspace);
  a.rowsum = d->a_rowsum;
  for (int q = 0; q < 2; ++q) {
    a.ra_ptr[q] = static_cast<const uint16_t*>(d->rowadd[q].ptr);
    a.ra_ld[q] = d->rowadd[q].ld;
    a.ra_T[q] = d->rowadd[q].rows_per_seq > 0 ? d->rowadd[q].rows_per_seq : 1;
    a.ra_seg[q] = d->rowadd[q].seg > 0 ? d->rowadd[q].seg : 1;
    a.ra_nseg[q] = d->rowadd[q].n_seg;
    a.ra_div[q] = d->rowadd[q].divisor;
  }
  a.act = d->act;
  a.aux = static_cast<uint16_t*>(d->aux);
  a.ld_aux = d->ld_aux;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (use_small(d)) {
    a.n_split = small_split(d);
    if (!d->a_trans && !d->b_trans) launch_small<true, true>(a, d->c_dtype, st);
    else if (!d->a_trans && d->b_trans) launch_small<true, false>(a, d->c_dtype, st);
    else if (d->a_trans && d->b_trans) launch_small<false, false>(a, d->c_dtype, st);
    else launch_small<false, true>(a, d->c_dtype, st);
    return check_launch("llattn_gemm");
  }
  // bf16 x Wᵀ (+ bias) (+ row addends) without K split or accumulation: the persistent kernel, one workgroup
  // per CU
  const int64_t c_bytes = ((int64_t)(d->M - 1) * d->ldc + d->N) * 2;
  const bool rowadd = d->rowadd[0].ptr || d->rowadd[1].ptr;
  if (!d->a_trans && !d->b_trans && S == 1 && d->c_dtype == LLATTN_BF16 && !d->accumulate &&
      c_bytes < (int64_t(1) << 31)) {
    // the pipeline fetches two 64-wide steps ahead: a contraction of one step runs as two, the second reading
    // zeros past K (every lane's chunk lies past it), which leaves the sums unchanged
    a.k_pairs = std::max(2, k_pairs);
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      cus = 256;
    const int tiles = a.tiles_m * a.tiles_n;
    if (a.act == LLATTN_ACT_GELU)
      hipLaunchKernelGGL(gemm_persistent_kernel<LLATTN_ACT_GELU>, dim3(std::min(tiles, cus)), dim3(256), 0, st, a);
    else if (ch.T)
      hipLaunchKernelGGL((gemm_persistent_kernel<LLATTN_ACT_NONE, true>), dim3(std::min(tiles, cus)), dim3(256), 0, st, a);
    else if (rowadd)
      hipLaunchKernelGGL((gemm_persistent_kernel<LLATTN_ACT_NONE, false, true>), dim3(std::min(tiles, cus)), dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL(gemm_persistent_kernel<LLATTN_ACT_NONE>, dim3(std::min(tiles, cus)), dim3(256), 0, st, a);
  } else if (ch.T) {
    return fail(LLATTN_ERR_UNSUPPORTED, "llattn_gemm: a split-head C of %lld bytes: the persistent kernel takes outputs "
                "below 2 GiB", (long long)c_bytes);
  } else if (rowadd && !d->b_trans) {
    return fail(LLATTN_ERR_UNSUPPORTED, "llattn_gemm: row addends with a k-contiguous B need the persistent kernel "
                "(no K split or accumulation, C below 2 GiB)");
  } else if (!d->a_trans && !d->b_trans) launch<true, true>(a, S, d->c_dtype, st);
  else if (!d->a_trans && d->b_trans) launch<true, false>(a, S, d->c_dtype, st);
  else if (d->a_trans && d->b_trans) launch<false, false>(a, S, d->c_dtype, st);
  else launch<false, true>(a, S, d->c_dtype, st);
  return check_launch("llattn_gemm");
}
