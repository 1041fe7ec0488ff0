/*
 * llattn.h -- C ABI of the MI355X (gfx950) local+latent attention kernels.
 *
 * Plain C: device pointers, element strides, sizes and an opaque stream
 * (a hipStream_t passed as void*).  No torch or HIP types appear here, so the
 * library binds from ctypes, cffi or any other FFI.  Every entry point is
 * asynchronous on the given stream, allocates nothing, keeps no global
 * mutable state apart from the calling thread's last error message, and
 * returns LLATTN_OK (0) or one of the status codes below; the message is
 * then available from llattn_last_error().
 *
 * Semantics are those of the reference PyTorch path LocalLatentAttention
 * (reference models.py:61-462); the entry points replace the launches of the
 * reference's fused op (reference kernels/llattn_op.py:34-181) and its
 * pooling helpers (reference llattn_triton.py:97-115, models.py:159-230).
 *
 * Tensor views (llattn_tensor) describe rows of head vectors
 * x[b][n][h][d] at ptr + b*sb + n*sn + h*sh + d (element strides; the head
 * dimension d is contiguous).  Rows and bases must be 16-byte aligned.
 */
#ifndef LLATTN_H
#define LLATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LLATTN_ABI_VERSION 8

/* status codes */
#define LLATTN_OK 0
#define LLATTN_ERR_SHAPE 1        /* inconsistent or non-positive sizes */
#define LLATTN_ERR_DTYPE 2        /* unknown dtype code */
#define LLATTN_ERR_LAYOUT 3       /* stride / alignment the kernels cannot read */
#define LLATTN_ERR_UNSUPPORTED 4  /* head dim or latent head dim outside the compiled set */
#define LLATTN_ERR_WORKSPACE 5    /* workspace missing or too small */
#define LLATTN_ERR_LAUNCH 6       /* the HIP runtime refused a launch */

/* dtype codes: storage type of every activation; accumulation is fp32 */
#define LLATTN_F32 0
#define LLATTN_BF16 1

/* pooling divisors */
#define LLATTN_DIV_COUNT 0  /* mean over the real tokens of a segment (reference models.py:182-200) */
#define LLATTN_DIV_SEG 1    /* sum / segment length, zero-padded mean (reference models.py:218-225) */
#define LLATTN_DIV_ONE 2    /* plain sum */

/* workspace kinds for llattn_workspace_size */
#define LLATTN_WS_LOCAL_BWD 0
#define LLATTN_WS_LATENT_BWD 1

typedef struct llattn_tensor {
  void* ptr;
  int64_t sb; /* batch stride */
  int64_t sn; /* row (token / latent / latent-query) stride */
  int64_t sh; /* head stride */
} llattn_tensor;

typedef struct llattn_shape {
  int32_t B, T;          /* batch, sequence length */
  int32_t H, Dh;         /* local heads, head dim (reference models.py:66-68); multiples of 8 up to 256 in bf16,
                            of 4 up to 128 in fp32 */
  int32_t Lh, Ldh;       /* latent heads, latent head dim (reference models.py:72-74); the same limits */
  int32_t window;        /* local window W (reference models.py:69) */
  int32_t block;         /* resolved local block size min(T, max(W, local_block_size)) (reference models.py:249) */
  int32_t chunk;         /* latent chunk ceil(T / min(latent_tokens, T)) (reference models.py:175-180) */
  int32_t n_chunks;      /* latent count (reference models.py:206-208) */
  int32_t q_block;       /* tokens per latent query: 1 token-wise, else min(T, qbs) (reference models.py:218) */
  int32_t n_q;           /* number of latent queries: T or ceil(T / q_block) */
  int32_t dtype;         /* LLATTN_F32 or LLATTN_BF16 */
  int32_t gate_per_head; /* 0: one gate vector shared by all heads (reference models.py:89-90); 1: [H][Dh] */
} llattn_shape;

/* ABI version of the loaded library (LLATTN_ABI_VERSION). */
int32_t llattn_abi_version(void);

/* Message of the calling thread's last failed call ("" when none). */
const char* llattn_last_error(void);

/* Bytes of workspace that llattn_local_gate_bwd (kind LLATTN_WS_LOCAL_BWD) or
 * llattn_latent_bwd (kind LLATTN_WS_LATENT_BWD) needs for this shape;
 * 0 on a bad shape (see llattn_last_error). */
size_t llattn_workspace_size(const llattn_shape* s, int32_t kind);

/* Segment pooling out[b][n][:] = sum_{t in segment n} x[b][t][:] / divisor.
 * Segments are [n*seg, min((n+1)*seg, T)).  Replaces _pool_to_latents
 * (reference models.py:159-214; LLATTN_DIV_COUNT) and _pool_query_blocks
 * (reference models.py:216-230; LLATTN_DIV_SEG); LLATTN_DIV_ONE folds
 * per-token gradients onto latent queries (backward of repeat_interleave,
 * reference models.py:398-412). */
int32_t llattn_pool_fwd(const void* x, int64_t x_sb, int64_t x_st, void* out, int64_t out_sb, int64_t out_sn,
                        int32_t B, int32_t T, int32_t D, int32_t seg, int32_t n_seg, int32_t divisor,
                        int32_t dtype, void* stream);

/* Backward of llattn_pool_fwd: dx[b][t][:] (+)= dpooled[b][t/seg][:] / divisor.
 * accumulate = 0 overwrites dx, 1 adds into it. */
int32_t llattn_pool_bwd(const void* dpooled, int64_t dp_sb, int64_t dp_sn, void* dx, int64_t dx_sb, int64_t dx_st,
                        int32_t B, int32_t T, int32_t D, int32_t seg, int32_t n_seg, int32_t divisor,
                        int32_t accumulate, int32_t dtype, void* stream);

/* Chunk-causal latent attention (reference models.py:361-375): query s of
 * latent head lh attends latents n < chunk_of(s) with scale 1/sqrt(Ldh);
 * queries with no latent output 0.  rq: [B][n_q][Lh][Ldh], gk/gv:
 * [B][n_chunks][Lh][Ldh], out: [B][n_q][Lh][Ldh]; lse: fp32 [B][Lh][n_q]
 * contiguous (-inf for empty rows), or NULL when no backward follows
 * (inference).  Replaces the latent half of the reference fused forward
 * launch (reference kernels/llattn_op.py:34-84). */
int32_t llattn_latent_fwd(const llattn_shape* s, const llattn_tensor* rq, const llattn_tensor* gk,
                          const llattn_tensor* gv, const llattn_tensor* out, float* lse, void* stream);

/* Backward of llattn_latent_fwd given dL = d(out) and the forward's lse:
 * writes drq, dgk, dgv (same layouts as rq, gk, gv).  The attention weights
 * are recomputed from lse in fp32.  Deterministic: per-tile partial sums in
 * the workspace, then an ordered reduction (no atomics).  Replaces the latent
 * part of the reference backward launches (reference kernels/llattn_op.py:87-181). */
int32_t llattn_latent_bwd(const llattn_shape* s, const llattn_tensor* rq, const llattn_tensor* gk,
                          const llattn_tensor* gv, const float* lse, const llattn_tensor* dout,
                          const llattn_tensor* drq, const llattn_tensor* dgk, const llattn_tensor* dgv,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Windowed local attention with the gate epilogue (reference models.py:232-305
 * and 416-438).  Query i attends keys max(0, i-W, floor(i/block)*block-W+1)
 * <= j <= i-1 with scale 1/sqrt(Dh); empty key sets give 0.  remote holds the
 * r_out output per latent query ([B][n_q][H][Dh]); token i reads row
 * i / q_block.  gate_l / gate_r: fp32 [Dh] (shared) or [H][Dh].  Writes
 * y = w*O + (1-w)*remote with w = sigmoid(gate_l.O - gate_r.remote),
 * o_local = O (pre-gate), lse [B][H][T] and w [B][H][T] (fp32, contiguous).
 * q/k/v/y/o_local: [B][T][H][Dh].  o_local, lse and w only feed the
 * backward: a forward-only call (inference, reference generate.py:188-190)
 * passes NULL for all three (o_local NULL or with a NULL ptr) and the kernel
 * writes y alone.  Replaces the local + gate half of the reference fused
 * forward launch (reference kernels/llattn_op.py:34-84). */
int32_t llattn_local_gate_fwd(const llattn_shape* s, const llattn_tensor* q, const llattn_tensor* k,
                              const llattn_tensor* v, const llattn_tensor* remote, const float* gate_l,
                              const float* gate_r, const llattn_tensor* y, const llattn_tensor* o_local,
                              float* lse, float* w, void* stream);

/* Backward of llattn_local_gate_fwd given dy: writes dq, dk, dv
 * ([B][T][H][Dh]), dremote per token ([B][T][H][Dh]; fold it onto latent
 * queries with llattn_pool_fwd(LLATTN_DIV_ONE) in macro-block mode) and the
 * fp32 gate gradients dgate_l / dgate_r ([H][Dh] with gate_per_head, else
 * [Dh]: the gradient of the shared gate, summed over heads).  dremote_colsum
 * (fp32 [H*Dh], or NULL) receives the fp32 sum of dremote over every token
 * and batch: the bias gradient of r_out, whose output is remote.  No
 * atomics; every sum runs in a fixed order.  Replaces the local + gate part
 * of the reference backward launches (reference kernels/llattn_op.py:87-181)
 * and r_out's bias gradient (reference models.py:84, 395). */
int32_t llattn_local_gate_bwd(const llattn_shape* s, const llattn_tensor* q, const llattn_tensor* k,
                              const llattn_tensor* v, const llattn_tensor* remote, const float* gate_l,
                              const float* gate_r, const llattn_tensor* o_local, const float* lse,
                              const float* w, const llattn_tensor* dy, const llattn_tensor* dq,
                              const llattn_tensor* dk, const llattn_tensor* dv, const llattn_tensor* dremote,
                              float* dgate_l, float* dgate_r, float* dremote_colsum, void* workspace,
                              size_t workspace_bytes, void* stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): llattn_local_gate_bwd with the same arguments and
 * results, minus the workspace.  Its scratch is a library-owned device array
 * of LLATTN_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends): the
 * gate partial sums, H*3*Dh*rows fp32, where rows = B * query segments for the
 * fused bf16 backward (W <= 64), B * ceil(T/128) for the bf16 wide-window
 * backward (W > 64, head dims up to 128) and B * ceil(T/64) otherwise; every
 * two-kernel path (all but the fused one) also holds dO_local and D there
 * (B*T*H*Dh elements, B*H*T fp32).  A shape that needs more returns
 * LLATTN_ERR_WORKSPACE.  Calls share their GPU's
 * array, so two calls that overlap on one GPU (different streams, threads or
 * processes) race; calls on one stream are ordered.  Allocates nothing. */
#define LLATTN_NOALLOC_SCRATCH_BYTES (8u << 20)
int32_t llattn_local_gate_bwd_noalloc(const llattn_shape* s, const llattn_tensor* q, const llattn_tensor* k,
                                      const llattn_tensor* v, const llattn_tensor* remote, const float* gate_l,
                                      const float* gate_r, const llattn_tensor* o_local, const float* lse,
                                      const float* w, const llattn_tensor* dy, const llattn_tensor* dq,
                                      const llattn_tensor* dk, const llattn_tensor* dv,
                                      const llattn_tensor* dremote, float* dgate_l, float* dgate_r,
                                      float* dremote_colsum, void* stream);

/* Projection GEMM on bf16 MFMA: C[m][n] = sum_k A(m,k) B(n,k) (+ bias[n])
 * (+ C[m][n] when accumulate).  A and B are bf16; each is stored
 * k-contiguous (A[M][K] / B[N][K], trans = 0) or m/n-contiguous
 * (A stored [K][M] / B stored [K][N], trans = 1), so the block's
 * forward (x W^T + b), input-gradient (dy W) and weight-gradient (dy^T x)
 * products all run without transpose copies.  C is bf16 or fp32; bias is
 * fp32 [N] or NULL.  Leading dimensions are in elements.  split_k = 0 picks
 * the number of K splits from the shape; more than one split writes fp32
 * partials to the workspace (llattn_gemm_workspace_size bytes) and sums them
 * in a fixed order.  Replaces the block's nn.Linear products and their
 * autograd backward (reference models.py:80-84, 315, 333-353, 395, 462). */
/* A bf16 matrix of rows broadcast onto token rows of C: C[m][n] += ptr[(m / rows_per_seq) * n_seg + t / seg][n]
 * / divisor with t = m % rows_per_seq (divisor as llattn_pool_bwd: LLATTN_DIV_COUNT, _SEG or _ONE).  The
 * backward of a pooling of the GEMM's input (reference models.py:159-230) added into its input gradient
 * before the bf16 rounding, without a separate pass over it.  ptr NULL: none. */
typedef struct llattn_gemm_rowadd {
  const void* ptr;  /* bf16 rows, 8-byte aligned */
  int64_t ld;       /* elements between rows, >= N, a multiple of 4 */
  int32_t rows_per_seq, seg, n_seg, divisor;
} llattn_gemm_rowadd;

/* Activation epilogues of llattn_gemm (bf16 C, a_trans = 0, no accumulation, no row addends), for the
 * FeedForward around the block (reference models.py:50-58: w2(gelu(w1 x)), F.gelu exact):
 *   LLATTN_ACT_GELU     with u = bf16(A B^T + bias) (the pre-activation):  C = bf16(gelu(u)), the
 *                       input of w2, and aux = bf16(gelu'(u)), what its backward multiplies by;
 *   LLATTN_ACT_MUL_AUX  C = bf16(bf16(A B...) * aux): the input gradient of w2 taken through the GELU
 *                       with the aux that LLATTN_ACT_GELU wrote.
 * gelu(u) = u Phi(u), gelu'(u) = Phi(u) + u phi(u) in fp32 on the bf16-rounded u (as bf16 autocast
 * evaluates F.gelu); gelu'(u) is then rounded to bf16 once more than autocast's backward does. */
#define LLATTN_ACT_NONE 0
#define LLATTN_ACT_GELU 1
#define LLATTN_ACT_MUL_AUX 2

/* Split-head storage of a bf16 matrix of token rows: a [rows][ld] matrix (rows = batch x T) keeps its first
 * n * dh columns as n head slabs per sequence, [batch][n][T][dh], followed by its other w = ld - n * dh
 * columns in a block of rows * w elements: packed rows [rows][w] (tail_dh = 0), or w / tail_dh slabs of
 * tail_dh columns, [batch][w / tail_dh][T][tail_dh] (tail_dh > 0).  Element (r, c), r = b T + t, sits at
 *   ((b n + c / dh) T + t) dh + c % dh                                  for c < n dh,
 *   rows n dh + r w + c'                                                 (tail_dh = 0),
 *   rows n dh + ((b w / tail_dh + c' / tail_dh) T + t) tail_dh + c' % tail_dh   (tail_dh > 0),
 * with c' = c - n dh.  The forward of the block's q|k|v (| token-wise latent query) projection writes it
 * this way (n = 3 H heads of dh = Dh, the latent queries as Lh slabs of tail_dh = Ldh), so that each head
 * of a sequence is one contiguous run for the attention kernels, which read q, k, v and the latent queries
 * by strides, in place of the packed [tokens][3 D (+ Ld)] matrix (reference models.py:315-316,
 * view(B, T, 3, H, Dh), and models.py:348-353, view(B, T, Lh, Ldh).transpose(1, 2)).  T = 0: plain row-major
 * storage. */
typedef struct llattn_heads_layout {
  int32_t T;        /* rows per sequence; 0: none */
  int32_t dh;       /* columns per head, a multiple of 8 */
  int32_t n;        /* head slabs per sequence */
  int32_t tail_dh;  /* 0: the other columns as packed rows; else their slab width, a multiple of 8 */
} llattn_heads_layout;

typedef struct llattn_gemm_desc {
  int32_t M, N, K;
  int32_t a_trans, b_trans;
  const void* A;
  int64_t lda;
  const void* B;
  int64_t ldb;
  void* C;
  int64_t ldc;
  int32_t c_dtype;     /* LLATTN_BF16 or LLATTN_F32 */
  int32_t accumulate;  /* 1: add into C */
  const float* bias;   /* fp32 [N] or NULL */
  int32_t split_k;     /* 0: automatic */
  float* a_rowsum;     /* fp32 [M] or NULL: also rowsum[m] = sum_k A(m,k), i.e. the bias gradient
                          sum_tokens dy of a weight-gradient product dy^T x, contracted against a
                          column of ones in place of the unused column N of the last tile, or, for
                          N % 256 == 0 (needs a_trans = 1 then), in extra products of the first tile
                          column; needs b_trans = 1 and fp32 C; overwritten, never accumulated */
  llattn_gemm_rowadd rowadd[2]; /* bf16 C, a_trans = 0, b_trans = 1 (input gradients) */
  int32_t act;                  /* LLATTN_ACT_* */
  void* aux;                    /* bf16 [M][ld_aux]: gelu' written (LLATTN_ACT_GELU) or read (_MUL_AUX) */
  int64_t ld_aux;
  /* bf16 C [M][ldc] stored split-head (the forward of a projection: a_trans = b_trans = 0, no K split,
     accumulation or activation). */
  llattn_heads_layout c_heads;
} llattn_gemm_desc;

size_t llattn_gemm_workspace_size(const llattn_gemm_desc* d);
int32_t llattn_gemm(const llattn_gemm_desc* d, void* workspace, size_t workspace_bytes, void* stream);

/* The same products in fp32: C = A Bᵀ (+ bias) (+ C with accumulate) with fp32 A, B and C (c_dtype
 * LLATTN_F32), the operand layouts of llattn_gemm (a_trans / b_trans, leading dimensions in elements,
 * 4-byte alignment) and optionally a_rowsum (any layout here); no K split, row addends, activation or
 * split-head C.  fp32 accumulation on v_mfma_f32_16x16x4_f32 in a fixed order, no workspace.  The
 * reference's nn.Linear products in fp32 (models.py:80-84, 315, 333-353, 395, 462) and their autograd,
 * for the fp32 module. */
int32_t llattn_gemm_f32(const llattn_gemm_desc* d, void* stream);

/* Column sums out[n] = sum_m x[m][n] in fp32 of a bf16 matrix x (M rows of
 * leading dimension ld): the bias gradient of a projection (sum over tokens of
 * its output gradient).  Two passes through a workspace of
 * llattn_colsum_workspace_size(M, N) bytes; deterministic.  Replaces the bias
 * gradients of the block's nn.Linear layers (reference models.py:80-84). */
size_t llattn_colsum_workspace_size(int32_t M, int32_t N);
int32_t llattn_colsum(const void* x, int64_t ld, int32_t M, int32_t N, float* out, void* workspace,
                      size_t workspace_bytes, void* stream);

/* fp32 arrays copied in one launch, each to bf16 (round to nearest even) or
 * fp32 per dst_dtype[i] (LLATTN_BF16 / LLATTN_F32): dst[i][0..n[i]) =
 * src[i][0..n[i]) for i < nseg <= LLATTN_CAST_MAX_SEGS; arrays aligned to
 * their element size (16-byte aligned ones move with vector loads/stores).  The per-forward fp32 -> bf16 weight casts that bf16 autocast makes
 * for every nn.Linear of the block (reference train.py:722, 982 around
 * models.py:80-84), and the concatenated biases of projections that share one
 * GEMM (qkv_proj + rq_proj), as one launch instead of one per array. */
#define LLATTN_CAST_MAX_SEGS 8
int32_t llattn_cast(int32_t nseg, const float* const* src, void* const* dst, const int64_t* n,
                    const int32_t* dst_dtype, void* stream);

/* llattn_cast, and for each segment i with dst_t[i] non-null also the transposed bf16 copy of the cast:
 * segment i is then a row-major fp32 [rows[i], n[i] / rows[i]] matrix (rows and columns multiples of 8,
 * src, dst and dst_t 16-byte aligned, bf16 output) and dst_t[i][c * ld_t[i] + r] = bf16(src[i][r * cols + c])
 * (ld_t[i] >= rows[i], a multiple of 8).  dst_t, ld_t and rows are nseg-entry arrays, or dst_t is NULL for
 * none.  The bf16 W^T copies that input gradients run on (dy W as dy (W^T)^T on the persistent GEMM, the
 * nn.Linear backward of reference models.py:80-84 under autocast), written while the cast reads W anyway:
 * one extra 2-byte write per element instead of an llattn_transpose pass in the backward. */
int32_t llattn_cast_transposed(int32_t nseg, const float* const* src, void* const* dst, const int64_t* n,
                               const int32_t* dst_dtype, void* const* dst_t, const int64_t* ld_t,
                               const int32_t* rows, void* stream);

/* dst[c][r] = src[r][c] for a bf16 matrix of rows x cols (both multiples of 8; 16-byte aligned, leading
 * dimensions in elements, multiples of 8).  The input gradient dy W of a projection runs as
 * dy (W^T)^T on the persistent GEMM (both operands k-contiguous) with this transposed copy of the bf16
 * weight (reference models.py:80-84, the nn.Linear backward under autocast). */
int32_t llattn_transpose(const void* src, int64_t ld_src, int32_t rows, int32_t cols, void* dst, int64_t ld_dst,
                         void* stream);

/* RMSNorm of the residual stream around the block (reference models.py:40-47,
 * F.rms_norm(x, (D,), w, eps), the LM's norm1 / norm2 / norm of reference
 * models.py:493-494, 513):
 *   y = x * rstd * w,  rstd[m] = 1 / sqrt(mean_d x[m][d]^2 + eps).
 * x, y: M rows of D elements (leading dimensions ldx / ldy in elements; rows
 * 16-byte (fp32) or 8-byte (bf16) aligned), each LLATTN_F32 or LLATTN_BF16 --
 * y in bf16 feeds the block's bf16 projections without a cast.  weight fp32
 * [D] (16-byte aligned); rstd fp32 [M] is written for the backward.
 * D must be a multiple of 4 and at most 4096.
 * With res non-null (fp32 x only): the residual add in front of the norm is
 * fused, as the LM block writes it (reference models.py:499-502,
 * x = x + attn(norm1(x)); x = x + ffn(norm2(x)) followed by the next norm):
 * xsum = x + res (fp32; res fp32 or bf16 per res_dtype, rows aligned as x's)
 * is written (xsum may be x itself) and y normalises xsum. */
int32_t llattn_rmsnorm_fwd(const void* x, int32_t x_dtype, int64_t ldx, const float* weight, int32_t M, int32_t D,
                           float eps, void* y, int32_t y_dtype, int64_t ldy, float* rstd, const void* res,
                           int32_t res_dtype, int64_t ldres, float* xsum, int64_t ldxsum, void* stream);

/* Backward of llattn_rmsnorm_fwd: dx (x's dtype) = rstd * (g - xh * mean_d(g xh)),
 * g = dy * w, xh = x * rstd; dweight (fp32 [D]) = sum over rows of dy * xh,
 * through a workspace of llattn_rmsnorm_workspace_size(M, D) bytes, added in a
 * fixed order (deterministic, no atomics).  Replaces the autograd backward of
 * the reference RMSNorm (reference models.py:40-47).  dres (x's dtype, may be
 * null; dx may be dres itself): the gradient reaching the norm's input through
 * the residual path, added to dx -- the backward of the fused residual add. */
size_t llattn_rmsnorm_workspace_size(int32_t M, int32_t D);
int32_t llattn_rmsnorm_bwd(const void* dy, int32_t dy_dtype, int64_t lddy, const void* x, int32_t x_dtype,
                           int64_t ldx, const float* rstd, const float* weight, int32_t M, int32_t D, void* dx,
                           int64_t lddx, float* dweight, const void* dres, int64_t lddres, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Cross entropy of bf16 logit rows and its gradient in one pass (the tied LM
 * head's loss, reference train.py:354-370: F.cross_entropy over [B*T, V]
 * logits in fp32 under autocast, ignore_index, and logits.argmax(-1) for the
 * accuracy metric; reference models.py:516-517, 576 for the head).  For each
 * of `rows` rows of V logits (leading dimension ld elements, 16-byte aligned
 * rows, V a multiple of 8, at most 65536):
 *   loss[r] = logsumexp(x_r) - x_r[t_r]   (0 where t_r == ignore_index,
 *             NaN where t_r lies outside [0, V) otherwise),
 *   pred[r] = first index of the row maximum (pred may be null),
 * and, when dlogits is non-null, dlogits[r][j] = (softmax(x_r)_j - [j == t_r])
 * * (*grad_scale) as bf16 (0 for ignored rows); dlogits may be the logits
 * buffer itself (in place) or a disjoint one.  targets: int64 [rows].
 * grad_scale: a device fp32 scalar (1 / valid rows for a mean).  One read and
 * one write of the logits; fixed-order reductions (deterministic). */
int32_t llattn_xent(const void* logits, int64_t ld, int32_t rows, int32_t V, const int64_t* targets,
                    int64_t ignore_index, float* loss, int32_t* pred, void* dlogits, int64_t ld_d,
                    const float* grad_scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LLATTN_H */
