// Device helpers shared by the gfx950 local+latent attention kernels.
//
// Storage types: float (fp32) or uint16_t holding bfloat16 bits.  All
// arithmetic accumulates in fp32.
//
// MFMA conventions (lane layouts checked on MI355X): a 64-lane wave is split
// into four lane groups g = lane/16 of 16 lanes, r = lane%16.
//   * 16x16 accumulator tile C[m][n]: lane (r, g) holds C[4g+i][r], i = 0..3.
//   * "row" products contract over a head dimension held row-major by both
//     operands (S = K Q^T, dP = V dO^T, ...).  Lane (r, g) supplies row r's
//     dims [g*DQ, (g+1)*DQ) where DQ = DHP/4 (DHP = head dim padded to a
//     multiple of 32); any consistent assignment of dims to MFMA k-slots
//     yields the same dot products.
//       bf16: v_mfma_f32_16x16x32_bf16, 8 dims per lane per step;
//       fp32: v_mfma_f32_16x16x4_f32,   1 dim per lane per step.
//   * "col" products contract over the 16 rows of a previous accumulator tile
//     (O^T = V^T P^T, dQ^T = K^T dS^T, ...).  The B operand is the lane's own
//     four accumulator values (k = 4g+i); the A operand is read from LDS as
//     four consecutive k of row m = r.
//       bf16: v_mfma_f32_16x16x16_bf16 (4 k per lane);
//       fp32: four v_mfma_f32_16x16x4_f32, step i uses k = 4g+i.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace llattn {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ float bf2f(uint16_t u) { return __uint_as_float(static_cast<uint32_t>(u) << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }

template <typename T>
__device__ __forceinline__ float to_f(T v) {
  if constexpr (std::is_same_v<T, float>) return v; else return bf2f(v);
}
template <typename T>
__device__ __forceinline__ T from_f(float v) {
  if constexpr (std::is_same_v<T, float>) return v; else return f2bf(v);
}
// value as it is stored (rounded to T) and read back
template <typename T>
__device__ __forceinline__ float round_t(float v) { return to_f<T>(from_f<T>(v)); }

// 16-byte vector of T
template <typename T> struct Vec16;
template <> struct Vec16<float> { static constexpr int N = 4; };
template <> struct Vec16<uint16_t> { static constexpr int N = 8; };

// ---- 4 consecutive elements <-> float[4] ------------------------------------
template <typename T>
__device__ __forceinline__ void load4(const T* p, float v[4]) {
  if constexpr (std::is_same_v<T, float>) {
    const float4 x = *reinterpret_cast<const float4*>(p);
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
  } else {
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    v[0] = __uint_as_float(x.x << 16); v[1] = __uint_as_float(x.x & 0xffff0000u);
    v[2] = __uint_as_float(x.y << 16); v[3] = __uint_as_float(x.y & 0xffff0000u);
  }
}
template <typename T>
__device__ __forceinline__ void store4(T* p, const float v[4]) {
  if constexpr (std::is_same_v<T, float>) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    uint2 x;
    x.x = static_cast<uint32_t>(f2bf(v[0])) | (static_cast<uint32_t>(f2bf(v[1])) << 16);
    x.y = static_cast<uint32_t>(f2bf(v[2])) | (static_cast<uint32_t>(f2bf(v[3])) << 16);
    *reinterpret_cast<uint2*>(p) = x;
  }
}
// 4 consecutive elements held as stored (8 bytes of bf16 / 16 bytes of fp32)
// so a prefetched row costs half the registers in bf16; zero when !valid.
__device__ __forceinline__ void unpack_bf16x4(uint2 v, float o[4]) {
  o[0] = __uint_as_float(v.x << 16); o[1] = __uint_as_float(v.x & 0xffff0000u);
  o[2] = __uint_as_float(v.y << 16); o[3] = __uint_as_float(v.y & 0xffff0000u);
}
template <typename T> struct Raw4;
template <> struct Raw4<float> {
  float4 v;
  __device__ __forceinline__ void load(const float* p, bool valid) {
    v = valid ? *reinterpret_cast<const float4*>(p) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  __device__ __forceinline__ void get(float o[4]) const { o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w; }
};
template <> struct Raw4<uint16_t> {
  uint2 v;
  __device__ __forceinline__ void load(const uint16_t* p, bool valid) {
    v = valid ? *reinterpret_cast<const uint2*>(p) : make_uint2(0u, 0u);
  }
  __device__ __forceinline__ void get(float o[4]) const {
    o[0] = __uint_as_float(v.x << 16); o[1] = __uint_as_float(v.x & 0xffff0000u);
    o[2] = __uint_as_float(v.y << 16); o[3] = __uint_as_float(v.y & 0xffff0000u);
  }
};

// ---- 16-byte copies (global <-> LDS) -----------------------------------------
__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }

// ---- row fragments ------------------------------------------------------------
template <typename T, int DQ> struct RowFrag;

template <int DQ> struct RowFrag<uint16_t, DQ> {
  static constexpr int N = DQ / 8;
  bf16x8 v[N];
  // row points at dim 0; dims >= Dh read as zero (Dh is a multiple of 8)
  __device__ __forceinline__ void load(const uint16_t* row, int g, int Dh, bool valid) {
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const int d = g * DQ + 8 * e;
      uint4 x = make_uint4(0, 0, 0, 0);
      if (valid && d < Dh) x = ld16(row + d);
      v[e] = __builtin_bit_cast(bf16x8, x);
    }
  }
  // LDS row already zero-padded to the full padded width
  __device__ __forceinline__ void load_lds(const uint16_t* row, int g) {
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = __builtin_bit_cast(bf16x8, ld16(row + g * DQ + 8 * e));
  }
};

template <int DQ> struct RowFrag<float, DQ> {
  static constexpr int N = DQ / 4;
  f32x4 v[N];
  __device__ __forceinline__ void load(const float* row, int g, int Dh, bool valid) {
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const int d = g * DQ + 4 * e;
      uint4 x = make_uint4(0, 0, 0, 0);
      if (valid && d < Dh) x = ld16(row + d);
      v[e] = __builtin_bit_cast(f32x4, x);
    }
  }
  __device__ __forceinline__ void load_lds(const float* row, int g) {
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = __builtin_bit_cast(f32x4, ld16(row + g * DQ + 4 * e));
  }
};

template <int DQ>
__device__ __forceinline__ f32x4 row_mma(const RowFrag<uint16_t, DQ>& a, const RowFrag<uint16_t, DQ>& b, f32x4 acc) {
#pragma unroll
  for (int e = 0; e < RowFrag<uint16_t, DQ>::N; ++e)
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v[e], b.v[e], acc, 0, 0, 0);
  return acc;
}
template <int DQ>
__device__ __forceinline__ f32x4 row_mma(const RowFrag<float, DQ>& a, const RowFrag<float, DQ>& b, f32x4 acc) {
#pragma unroll
  for (int e = 0; e < RowFrag<float, DQ>::N; ++e)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[e][c], b.v[e][c], acc, 0, 0, 0);
  return acc;
}

// ---- col products: A = 4 consecutive k of row m (LDS), B = lane's 4 values ----
__device__ __forceinline__ f32x4 col_mma(const uint16_t* a, const float b[4], f32x4 acc) {
  const i16x4 av = *reinterpret_cast<const i16x4*>(a);
  i16x4 bv;
  bv[0] = static_cast<short>(f2bf(b[0]));
  bv[1] = static_cast<short>(f2bf(b[1]));
  bv[2] = static_cast<short>(f2bf(b[2]));
  bv[3] = static_cast<short>(f2bf(b[3]));
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, bv, acc, 0, 0, 0);
}
__device__ __forceinline__ f32x4 col_mma(const float* a, const float b[4], f32x4 acc) {
  const f32x4 av = *reinterpret_cast<const f32x4*>(a);
#pragma unroll
  for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], b[i], acc, 0, 0, 0);
  return acc;
}

// ---- wave reductions over the four lane groups (same r) ------------------------
__device__ __forceinline__ float sum_groups(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}
__device__ __forceinline__ float max_groups(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}
// Workgroup barrier that orders LDS only: the fences are limited to the local
// address space, so the wave waits for its own LDS operations (lgkmcnt(0)) but
// global loads and stores stay in flight across it (a full __syncthreads also
// waits for vmcnt(0), which would drain every prefetch issued before it).  Only
// for kernels in which no wave reads global memory that another wave of the
// workgroup wrote.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// sum over the 16 lanes of a group (same g), valid in the group's last lane
// (r = 15): a DPP row_shr ladder (VALU; out-of-row sources read 0)
__device__ __forceinline__ float sum_rows16_last(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x111, 0xf, 0xf, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x112, 0xf, 0xf, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x114, 0xf, 0xf, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x118, 0xf, 0xf, true));
  return x;
}
// sum over each aligned group of 8 lanes, in every lane of the group: quad
// swaps (quad_perm [1,0,3,2], [2,3,0,1]) then row_half_mirror (lane i <- 7-i)
__device__ __forceinline__ float sum_lanes8(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xf, 0xf, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4E, 0xf, 0xf, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x141, 0xf, 0xf, true));
  return x;
}
// sum over the 16 lanes of a group (same g)
__device__ __forceinline__ float sum_rows16(float x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 8);
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- LDS staging of 64-row tiles (256 threads) --------------------------------
constexpr int kTP = 68;  // pitch (elements) of transposed tiles [dim][64 rows + 4]
template <typename T> constexpr int kRowPad = std::is_same_v<T, float> ? 4 : 8;

// Rows [r0, r0+64) of a row view (row stride st) into LDS row-major [64][P];
// rows >= r_end and dims >= Dh are zero.  Consecutive threads take consecutive
// 16-byte chunks of a row (coalesced reads).
template <typename T, int DHP, int P>
__device__ __forceinline__ void stage_rows(T* lds, const T* base, int64_t st, int r0, int r_end, int Dh) {
  constexpr int V = Vec16<T>::N, CPR = DHP / V;
  for (int c = threadIdx.x; c < 64 * CPR; c += 256) {
    const int row = c / CPR, col = (c % CPR) * V, rr = r0 + row;
    uint4 x = make_uint4(0, 0, 0, 0);
    if (rr < r_end && col < Dh) x = ld16(base + (int64_t)rr * st + col);
    st16(lds + row * P + col, x);
  }
}

// ---- col products with A read from a row-major LDS tile ------------------------
// base = &tile[k0][m0] of a row-major tile with pitch P: A[m][k] = tile[k0 + k][m0 + m].
// bf16: one ds_read_b64_tr_b16 gives lane (r, g) the four elements
// tile[k0 + 4g + i][m0 + r], i = 0..3 (within each 16-lane group, lane j
// supplies the address of row 4g + j/4, columns 4(j%4) .. 4(j%4)+3).
// two floats -> packed bf16 pair (round to nearest even; one v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}
__device__ __forceinline__ i16x4 pack_bf16x4(const float b[4]) {
  const uint2 u = make_uint2(pack_bf16x2(b[0], b[1]), pack_bf16x2(b[2], b[3]));
  return __builtin_bit_cast(i16x4, u);
}
// col_mma_rm with the lane's four B values already packed (convert once, use for every t)
template <int P>
__device__ __forceinline__ f32x4 col_mma_rm(const uint16_t* base, const i16x4 bv, f32x4 acc) {
  typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const uint16_t* p = base + (4 * g + (j >> 2)) * P + 4 * (j & 3);
  const bf16x4 av = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4*)(p));
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, av), bv, acc, 0, 0, 0);
}
template <int P>
__device__ __forceinline__ f32x4 col_mma_rm(const uint16_t* base, const float b[4], f32x4 acc) {
  typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const uint16_t* p = base + (4 * g + (j >> 2)) * P + 4 * (j & 3);
  const bf16x4 av = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4*)(p));
  i16x4 bv;
  bv[0] = static_cast<short>(f2bf(b[0]));
  bv[1] = static_cast<short>(f2bf(b[1]));
  bv[2] = static_cast<short>(f2bf(b[2]));
  bv[3] = static_cast<short>(f2bf(b[3]));
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, av), bv, acc, 0, 0, 0);
}
// fp32: four scalar LDS reads tile[k0 + 4g + i][m0 + r]; step i contracts k = 4g + i.
template <int P>
__device__ __forceinline__ f32x4 col_mma_rm(const float* base, const float b[4], f32x4 acc) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const float* p = base + (4 * g) * P + r;
#pragma unroll
  for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(p[i * P], b[i], acc, 0, 0, 0);
  return acc;
}

// ---- register-staged 64-row tiles ---------------------------------------------
// A tile is copied global -> registers -> LDS in two steps so that every global
// load of the tile is in flight at once (and the next tile's loads can overlap
// the current tile's MFMA work): load() issues the loads, store*() writes LDS.
//
// RowTile: row-major [64][P] copy; consecutive threads take consecutive 16-byte
// chunks of a row (coalesced reads).  Rows >= r_end and dims >= Dh are zero.
template <typename T, int DHP, int NTHR = 256>
struct RowTile {
  static constexpr int V = Vec16<T>::N, CPR = DHP / V, TASKS = 64 * CPR, IT = (TASKS + NTHR - 1) / NTHR;
  uint4 x[IT];
  __device__ __forceinline__ void load(const T* base, int64_t st, int r0, int r_end, int Dh) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int task = threadIdx.x + NTHR * it, row = task / CPR, col = (task % CPR) * V, rr = r0 + row;
      x[it] = make_uint4(0, 0, 0, 0);
      if (task < TASKS && rr < r_end && col < Dh) x[it] = ld16(base + (int64_t)rr * st + col);
    }
  }
  // rows (r0 + i) / div of the view (one row per latent query in macro-block
  // mode); tile rows with r0 + i >= r_end are zero
  __device__ __forceinline__ void load_div(const T* base, int64_t st, int r0, int r_end, int div, int Dh) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int task = threadIdx.x + NTHR * it, row = task / CPR, col = (task % CPR) * V, rr = r0 + row;
      x[it] = make_uint4(0, 0, 0, 0);
      if (task < TASKS && rr < r_end && col < Dh) x[it] = ld16(base + (int64_t)(rr / div) * st + col);
    }
  }
  template <int P>
  __device__ __forceinline__ void store(T* lds) const {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int task = threadIdx.x + NTHR * it, row = task / CPR, col = (task % CPR) * V;
      if (task < TASKS) st16(lds + row * P + col, x[it]);
    }
  }
};

// ---- buffer loads (range-checked: an offset past the resource's extent reads zero) ----
constexpr uint32_t kOffOOB = 0x80000000u;  // an offset beyond every extent used here (< 2 GiB)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int64_t bytes) {
  const int n = bytes <= 0 ? 0 : (bytes >= (int64_t)kOffOOB ? (int)(kOffOOB - 16) : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, n, 0x00020000);
}
// kStream: the non-temporal cache policy (nt) for rows a kernel reads once with whole-row 16-byte loads.
// Such rows then do not push out of L2 the lines that stores are still filling (an output row of one
// head shares its first and last 128-byte lines with the neighbouring heads' rows, written by other
// workgroups).  Not for rows that several load instructions or workgroups read in turn: the line is
// then fetched again.
constexpr int kCached = 0, kStream = 2;
template <int POLICY = kCached>
__device__ __forceinline__ uint4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POLICY));
}
template <int POLICY = kCached>
__device__ __forceinline__ uint2 buf_ld8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, POLICY));
}

// BufTile: a bf16 RowTile read with buffer loads.  Each thread's byte offset
// within a tile is a fixed function of its index and the row stride; the
// tile's rows come from a resource that ends with the last valid row, so
// rows past the end and padding dims read as zero without branches.
// Offsets are 32-bit: 64 rows of the view must span less than 2 GiB.
template <int DHP, int NTHR>
struct BufTile {
  static constexpr int CPR = DHP / 8, TASKS = 64 * CPR, IT = (TASKS + NTHR - 1) / NTHR;
  uint4 x[IT];
  // rows [r0, r_end) of the view at base (row stride st elements), with cache policy POLICY
  template <int POLICY = kCached>
  __device__ __forceinline__ void load(const uint16_t* base, int st, int r0, int r_end, int Dh, int tid) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(base + (int64_t)r0 * st, ((int64_t)(r_end - r0 - 1) * st + Dh) * 2);
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int task = tid + NTHR * it, row = task / CPR, col = (task % CPR) * 8;
      x[it] = buf_ld16<POLICY>(rs, (task < TASKS && col < Dh) ? (uint32_t)(row * st + col) * 2u : kOffOOB);
    }
  }
  // rows (r0 + i) / div of the view for r0 + i < r_end (one row per latent query of div tokens); tile rows
  // past r_end read zero
  template <int POLICY = kCached>
  __device__ __forceinline__ void load_div(const uint16_t* base, int st, int r0, int r_end, int div, int Dh,
                                           int tid) {
    const int b0 = r0 / div, b_end = r_end > r0 ? (r_end - 1) / div + 1 : b0;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(base + (int64_t)b0 * st, ((int64_t)(b_end - b0 - 1) * st + Dh) * 2);
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int task = tid + NTHR * it, row = task / CPR, col = (task % CPR) * 8, rr = r0 + row;
      x[it] = buf_ld16<POLICY>(rs, (task < TASKS && rr < r_end && col < Dh) ? (uint32_t)((rr / div - b0) * st + col) * 2u
                                                                           : kOffOOB);
    }
  }
  // tid: the thread's index among the NTHR threads that share the tile
  template <int P>
  __device__ __forceinline__ void store(uint16_t* lds, int tid) const {
    // the thread's LDS offsets are recomputed here rather than kept live across a caller's loop
    int zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int task = tid + zero + NTHR * it, row = task / CPR, col = (task % CPR) * 8;
      if (task < TASKS) st16(lds + row * P + col, x[it]);
    }
  }
};

// Coalesced copy of a row-major 64-row LDS tile (pitch P) to global rows
// r0 + i (row stride st) for r0 + i < r_end and dims < Dh.
template <typename T, int DHP, int P, int NTHR = 256>
__device__ __forceinline__ void store_tile(T* base, int64_t st, const T* lds, int r0, int r_end, int Dh) {
  constexpr int V = Vec16<T>::N, CPR = DHP / V, TASKS = 64 * CPR, IT = (TASKS + NTHR - 1) / NTHR;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int task = threadIdx.x + NTHR * it, row = task / CPR, col = (task % CPR) * V, rr = r0 + row;
    if (task < TASKS && rr < r_end && col < Dh) st16(base + (int64_t)rr * st + col, ld16(lds + row * P + col));
  }
}

// TransTile: the rows stored transposed into LDS [DHP][kTP] (row index
// contiguous), and optionally row-major too.  The row index varies fastest
// across threads so the transposed writes are whole dwords without bank
// conflicts: a bf16 thread holds a pair of rows and packs the two rows'
// elements of one dim into a dword.
template <typename T, int DHP>
struct TransTile {
  static constexpr bool kF32 = std::is_same_v<T, float>;
  static constexpr int V = Vec16<T>::N, CPR = DHP / V, RPT = kF32 ? 1 : 2, NR = 64 / RPT;
  static constexpr int TASKS = NR * CPR, IT = (TASKS + 255) / 256;
  uint4 x[IT][RPT];
  __device__ __forceinline__ void load(const T* base, int64_t st, int r0, int r_end, int Dh) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int task = threadIdx.x + 256 * it, row = RPT * (task % NR), col = (task / NR) * V, rr = r0 + row;
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        x[it][j] = make_uint4(0, 0, 0, 0);
        if (task < TASKS && col < Dh && rr + j < r_end) x[it][j] = ld16(base + (int64_t)(rr + j) * st + col);
      }
    }
  }
  template <int P>
  __device__ __forceinline__ void store_rows(T* lds) const {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int task = threadIdx.x + 256 * it, row = RPT * (task % NR), col = (task / NR) * V;
      if (task < TASKS) {
#pragma unroll
        for (int j = 0; j < RPT; ++j) st16(lds + (row + j) * P + col, x[it][j]);
      }
    }
  }
  __device__ __forceinline__ void store_t(T* lds_t) const {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int task = threadIdx.x + 256 * it, row = RPT * (task % NR), col = (task / NR) * V;
      if (task >= TASKS) continue;
      if constexpr (kF32) {
        const uint4 v = x[it][0];
        lds_t[(col + 0) * kTP + row] = __uint_as_float(v.x);
        lds_t[(col + 1) * kTP + row] = __uint_as_float(v.y);
        lds_t[(col + 2) * kTP + row] = __uint_as_float(v.z);
        lds_t[(col + 3) * kTP + row] = __uint_as_float(v.w);
      } else {
        const uint4 x0 = x[it][0], x1 = x[it][1];
        const uint32_t a[4] = {x0.x, x0.y, x0.z, x0.w}, b[4] = {x1.x, x1.y, x1.z, x1.w};
        uint32_t* dst = reinterpret_cast<uint32_t*>(lds_t + col * kTP + row);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dst[(2 * j) * (kTP / 2)] = (a[j] & 0xffffu) | (b[j] << 16);
          dst[(2 * j + 1) * (kTP / 2)] = (a[j] >> 16) | (b[j] & 0xffff0000u);
        }
      }
    }
  }
};

// ---- online softmax + PV for one 16-key sub-tile -----------------------------
// s: S^T[key 4g+i][query r] (raw scores); ok[i]: key 4g+i visible to query r.
// Updates the running max / partial sum of query r (max shared by the four
// lane groups) and O^T += V^T P^T with vt = &Vt[r][16*sub + 4g] (LDS, pitch kTP).
template <int NT, typename T>
__device__ __forceinline__ void online_softmax_pv(const f32x4& s, const bool ok[4], float scale_log2, float& m_run,
                                                  float& l_run, f32x4 (&acc)[NT], const T* vt) {
  float sv[4], mloc = kNegInf;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sv[i] = ok[i] ? s[i] * scale_log2 : kNegInf;
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
  for (int t = 0; t < NT; ++t) {
    acc[t] *= alpha;
    acc[t] = col_mma(vt + 16 * t * kTP, pv, acc[t]);
  }
}

// Workgroups are dispatched round-robin over the 8 XCDs; remap so that each
// XCD receives a contiguous range of logical tiles (neighbouring query tiles
// of one head share K/V rows, which then stay in that XCD's L2).  XCD x holds
// the ids x, x+8, ... < nblocks: nblocks/8 of them, one more when x < nblocks%8,
// so its range starts after the x ranges before it.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  const int x = bid & 7, q = nblocks >> 3, r = nblocks & 7;
  return x * q + min(x, r) + (bid >> 3);
}

// First key of query i (inclusive); the last is i-1.  The reference runs SDPA
// per block of `bs` queries over keys [max(0, q0-W+1), q_end) with the mask
// 0 < i-j <= W (reference models.py:249-292).
__device__ __forceinline__ int key_lo(int i, int W, int bs) {
  const int q0 = (i / bs) * bs;
  return max(max(0, i - W), q0 - W + 1);
}

}  // namespace llattn
