"""CPU oracle for the local+latent attention block (TEST INFRASTRUCTURE ONLY).

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it.  The shipped op (``local-latent-attention_amd``) must never route through
it; on a box without the HIP library the product raises instead.

It restates, in float64 numpy with an explicit hand-derived backward, the
semantics of the reference PyTorch path ``LocalLatentAttention``
(``/root/reference/models.py:61-462``).  Every function cites the reference
lines it follows.  The backward is NOT autograd: it is written out from the
forward equations so that finite differences of :func:`module_forward` check
it independently.

Pinning (what makes this restatement trustworthy; the tests named live in
``tests/test_oracle.py``):

* golden vectors written by importing the reference ``models.py`` on CPU
  (``tests/golden/make_golden.py``) pin the end-to-end forward, every
  parameter/input gradient, the local key set with the block-start quirk,
  both pooling modes and the macro-block expansion, at shapes chosen to hit
  every edge case (remainder chunk, partial query block, W=1, T < latent
  count, single block);
* brute force: the local key set against a literal replay of the
  reference's block loop; the banded attention against dense [T,T] masked
  softmax; pooling against per-chunk python means;
* closed forms: W >= T and bs >= T gives strictly-causal attention; chunk
  size 1 gives strictly-causal latent attention over rkv_proj(x); chunk-0
  tokens get ``remote = r_out.bias``; gate saturation gives the pure
  local/remote branch; ``w_l + w_r = 1``;
* the backward: central finite differences of :func:`module_forward` in
  float64 for x and every parameter.

No function here is "parity unpinned".
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

# --------------------------------------------------------------------------
# shape resolution
# --------------------------------------------------------------------------


@dataclass(frozen=True)
class BlockShape:
    """Hyper-parameters of one attention block.

    Field meaning follows ``ModelConfig`` (``models.py:21-37``): ``window`` is
    ``local_window``, ``latent_tokens`` the latent-count upper bound,
    ``latent_d_model``/``latent_heads`` the latent width and head count.
    """

    d_model: int
    n_heads: int
    window: int
    local_block_size: int = 256
    latent_tokens: int = 16
    latent_d_model: int = 64
    latent_heads: int = 2
    latent_query_block_size: int = 0

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads

    @property
    def latent_head_dim(self) -> int:
        return self.latent_d_model // self.latent_heads

    @property
    def macro(self) -> bool:
        # models.py:343 -- macro-block queries only when the block size is > 1
        return self.latent_query_block_size > 1


@dataclass(frozen=True)
class SeqLayout:
    """Index maps of one sequence length (all integers, shared by every batch row)."""

    T: int
    bs: int            # local query-block size, models.py:249
    chunk: int         # latent pooling chunk, models.py:175-180
    n_chunks: int      # actual latent count, models.py:206-208
    chunk_ids: np.ndarray   # token -> chunk, models.py:211-212
    qb: int            # latent query block (1 in token-wise mode), models.py:218
    n_q: int           # number of latent queries
    q_chunk_ids: np.ndarray  # latent query -> causal latent limit, models.py:226-230
    key_lo: np.ndarray  # first allowed local key per query (inclusive)
    key_hi: np.ndarray  # last allowed local key per query (inclusive)


def seq_layout(shape: BlockShape, T: int) -> SeqLayout:
    """Resolve every integer index map for sequence length ``T``.

    * local block size ``bs = min(T, max(W, local_block_size))`` -- models.py:249
    * key set of query i: the reference runs SDPA per query block
      ``[q0, q0+bs)`` over keys ``[max(0, q0-W+1), q_end)`` with the mask
      ``0 < i-j <= W`` (models.py:251-292), so query i sees
      ``max(0, i-W, q0(i)-W+1) <= j <= i-1``;
    * chunking: ``chunk = ceil(T / min(latent_tokens, T))``; the last chunk
      may be partial; ``chunk_ids = i // chunk`` (models.py:175-212);
    * macro-block queries: ``qb = min(T, qbs)``, ``n_q = ceil(T/qb)``; a block
      takes the smallest chunk id of its tokens, i.e. that of its first token
      (models.py:216-230).
    """
    if T <= 0:
        raise ValueError("seq_len must be positive")  # models.py:171-172
    if shape.window <= 0:
        raise ValueError("local_window must be positive")  # models.py:246-247
    target = min(shape.latent_tokens, T)
    if target <= 0:
        raise ValueError("latent_tokens must be positive")  # models.py:176-177
    chunk = -(-T // target)
    n_chunks = T // chunk + (1 if T % chunk else 0)
    tok = np.arange(T, dtype=np.int64)
    chunk_ids = np.minimum(tok // chunk, n_chunks - 1)
    bs = min(T, max(shape.window, shape.local_block_size))
    q0 = (tok // bs) * bs
    key_lo = np.maximum(np.maximum(0, tok - shape.window), q0 - shape.window + 1)
    key_hi = tok - 1
    if shape.macro:
        qb = min(T, shape.latent_query_block_size)
        n_q = -(-T // qb)
        q_chunk_ids = np.array([chunk_ids[s * qb: min((s + 1) * qb, T)].min() for s in range(n_q)],
                               dtype=np.int64)
    else:
        qb, n_q, q_chunk_ids = 1, T, chunk_ids.copy()
    return SeqLayout(T, bs, chunk, n_chunks, chunk_ids, qb, n_q, q_chunk_ids, key_lo, key_hi)


# --------------------------------------------------------------------------
# parameters
# --------------------------------------------------------------------------

PARAM_NAMES = (
    "qkv_proj.weight", "qkv_proj.bias",
    "rq_proj.weight", "rq_proj.bias",
    "rkv_proj.weight", "rkv_proj.bias",
    "r_out.weight", "r_out.bias",
    "out.weight", "out.bias",
    "gate_local.weight", "gate_remote.weight",
)


def param_shapes(shape: BlockShape) -> dict[str, tuple[int, ...]]:
    """Parameter names and shapes of ``LocalLatentAttention`` (models.py:80-90)."""
    D, Ld, Dh = shape.d_model, shape.latent_d_model, shape.head_dim
    return {
        "qkv_proj.weight": (3 * D, D), "qkv_proj.bias": (3 * D,),
        "rq_proj.weight": (Ld, D), "rq_proj.bias": (Ld,),
        "rkv_proj.weight": (2 * Ld, D), "rkv_proj.bias": (2 * Ld,),
        "r_out.weight": (D, Ld), "r_out.bias": (D,),
        "out.weight": (D, D), "out.bias": (D,),
        "gate_local.weight": (1, Dh), "gate_remote.weight": (1, Dh),
    }


# --------------------------------------------------------------------------
# forward pieces
# --------------------------------------------------------------------------


def pool_segments(x: np.ndarray, seg: int, n_seg: int, divisor: str) -> np.ndarray:
    """Sum x[B,T,D] over consecutive segments of ``seg`` tokens.

    ``divisor='count'`` averages over the real tokens of each segment
    (``_pool_to_latents``, models.py:182-200); ``divisor='seg'`` divides every
    segment, including a partial last one, by ``seg`` -- the zero-padded mean
    of ``_pool_query_blocks`` (models.py:218-225); ``divisor='one'`` returns
    plain sums.
    """
    B, T, D = x.shape
    out = np.zeros((B, n_seg, D), dtype=x.dtype)
    for n in range(n_seg):
        a, b = n * seg, min((n + 1) * seg, T)
        s = x[:, a:b, :].sum(axis=1)
        if divisor == "count":
            s = s / (b - a)
        elif divisor == "seg":
            s = s / seg
        out[:, n, :] = s
    return out


def local_attention(q, k, v, lay: SeqLayout, qblk: int = 256):
    """Windowed strictly-past attention of ``_local_attention`` (models.py:232-276).

    q, k, v: [B, H, T, Dh].  Scale ``1/sqrt(Dh)`` (SDPA default).  A query
    with an empty key set (token 0; block starts when W == 1) outputs 0, as
    torch's SDPA does for a fully -inf masked row.  Returns (O, LSE) with
    LSE = -inf for empty rows.  Banded: queries are processed in blocks of
    ``qblk`` against the keys that block can reach.
    """
    B, H, T, Dh = q.shape
    scale = 1.0 / math.sqrt(Dh)
    O = np.zeros_like(q)
    LSE = np.full((B, H, T), -np.inf, dtype=q.dtype)
    for a in range(0, T, qblk):
        b = min(a + qblk, T)
        ka = int(lay.key_lo[a:b].min())
        kb = int(lay.key_hi[a:b].max()) + 1
        if kb <= ka:
            continue
        j = np.arange(ka, kb)
        allowed = (j[None, :] >= lay.key_lo[a:b, None]) & (j[None, :] <= lay.key_hi[a:b, None])
        s = np.einsum("bhid,bhjd->bhij", q[:, :, a:b], k[:, :, ka:kb]) * scale
        s = np.where(allowed, s, -np.inf)
        m = s.max(axis=-1, keepdims=True)
        m_safe = np.where(np.isfinite(m), m, 0.0)
        p = np.exp(s - m_safe)
        l = p.sum(axis=-1, keepdims=True)
        has = l > 0
        p = np.where(has, p / np.where(has, l, 1.0), 0.0)
        O[:, :, a:b] = np.einsum("bhij,bhjd->bhid", p, v[:, :, ka:kb])
        LSE[:, :, a:b] = np.where(has[..., 0], (m_safe + np.log(np.where(has, l, 1.0)))[..., 0], -np.inf)
    return O, LSE


def latent_attention(rq, gk, gv, q_chunk_ids):
    """Chunk-causal latent attention (models.py:361-375).

    rq: [B, Lh, Q, Ldh]; gk, gv: [B, Lh, Nc, Ldh].  Query s sees latents
    ``n < q_chunk_ids[s]``; a query with none (chunk 0) outputs 0.
    Returns (L, P) with P the [B, Lh, Q, Nc] attention weights.
    """
    Ldh = rq.shape[-1]
    s = np.einsum("bhsd,bhnd->bhsn", rq, gk) / math.sqrt(Ldh)
    n = np.arange(gk.shape[2])
    allowed = n[None, :] < q_chunk_ids[:, None]
    s = np.where(allowed, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(s - m_safe)
    l = p.sum(axis=-1, keepdims=True)
    has = l > 0
    P = np.where(has, p / np.where(has, l, 1.0), 0.0)
    return np.einsum("bhsn,bhnd->bhsd", P, gv), P


def gate_mix(O_l, R_tok, g_l, g_r):
    """Shared-weight two-branch gate (models.py:416-438).

    O_l, R_tok: [B, H, T, Dh]; g_l, g_r: [Dh] (one ``Linear(Dh,1)`` per branch
    shared by all heads, models.py:89-90).  Returns (Y, w_local, s_l, s_r)
    with ``w_local = exp(s_l-m)/(exp(s_l-m)+exp(s_r-m))``.
    """
    s_l = O_l @ g_l
    s_r = R_tok @ g_r
    m = np.maximum(s_l, s_r)
    e_l = np.exp(s_l - m)
    e_r = np.exp(s_r - m)
    w = e_l / (e_l + e_r)
    wr = e_r / (e_l + e_r)
    Y = w[..., None] * O_l + wr[..., None] * R_tok
    return Y, w, s_l, s_r


def _linear(x, W, b):
    return x @ W.T + b


def module_forward(params: dict, x: np.ndarray, shape: BlockShape, keep: bool = False):
    """Forward of ``LocalLatentAttention`` (models.py:307-462) in float64.

    ``params`` maps :data:`PARAM_NAMES` to arrays; x is [B, T, D].  With
    ``keep=True`` also returns the dict of intermediates the backward uses.
    """
    B, T, D = x.shape
    H, Dh = shape.n_heads, shape.head_dim
    Lh, Ldh, Ld = shape.latent_heads, shape.latent_head_dim, shape.latent_d_model
    lay = seq_layout(shape, T)

    qkv = _linear(x, params["qkv_proj.weight"], params["qkv_proj.bias"]).reshape(B, T, 3, H, Dh)
    q, k, v = (qkv[:, :, i].transpose(0, 2, 1, 3) for i in range(3))       # models.py:315-319

    pooled = pool_segments(x, lay.chunk, lay.n_chunks, "count")            # models.py:325
    gkgv = _linear(pooled, params["rkv_proj.weight"], params["rkv_proj.bias"])
    gkgv5 = gkgv.reshape(B, lay.n_chunks, 2, Lh, Ldh)
    gk = gkgv5[:, :, 0].transpose(0, 2, 1, 3)                             # models.py:333-342
    gv = gkgv5[:, :, 1].transpose(0, 2, 1, 3)
    if shape.macro:
        qsrc = pool_segments(x, lay.qb, lay.n_q, "seg")                     # models.py:343-344
    else:
        qsrc = x
    rq_flat = _linear(qsrc, params["rq_proj.weight"], params["rq_proj.bias"])  # models.py:348
    rq = rq_flat.reshape(B, lay.n_q, Lh, Ldh).transpose(0, 2, 1, 3)

    O_l, LSE = local_attention(q, k, v, lay)                               # models.py:355
    L, P = latent_attention(rq, gk, gv, lay.q_chunk_ids)                  # models.py:361-375
    L_flat = L.transpose(0, 2, 1, 3).reshape(B, lay.n_q, Ld)              # models.py:392-394
    R_q = _linear(L_flat, params["r_out.weight"], params["r_out.bias"])     # models.py:395
    tok_q = np.arange(T) // lay.qb                                          # models.py:398-414
    R_tok = R_q[:, tok_q].reshape(B, T, H, Dh).transpose(0, 2, 1, 3)
    Y, w, s_l, s_r = gate_mix(O_l, R_tok, params["gate_local.weight"][0], params["gate_remote.weight"][0])
    Y_flat = Y.transpose(0, 2, 1, 3).reshape(B, T, D)                     # models.py:438
    out = _linear(Y_flat, params["out.weight"], params["out.bias"])        # models.py:462
    if not keep:
        return out
    cache = dict(lay=lay, q=q, k=k, v=v, pooled=pooled, gk=gk, gv=gv, qsrc=qsrc, rq=rq,
                 O_l=O_l, LSE=LSE, L=L, P=P, L_flat=L_flat, R_q=R_q, R_tok=R_tok, Y=Y,
                 Y_flat=Y_flat, w=w, tok_q=tok_q)
    return out, cache


# --------------------------------------------------------------------------
# backward (hand-derived; checked by finite differences of module_forward)
# --------------------------------------------------------------------------


def gate_backward(dY, O_l, R_tok, w, g_l, g_r):
    """Backward of :func:`gate_mix`.  All [B,H,T,Dh] except w [B,H,T].

    delta = w(1-w) * dY.(O_l - R);  dO_l = w dY + delta g_l;
    dR = (1-w) dY - delta g_r;  dg_l = sum delta O_l;  dg_r = -sum delta R.
    """
    delta = w * (1.0 - w) * np.einsum("bhtd,bhtd->bht", dY, O_l - R_tok)
    dO = w[..., None] * dY + delta[..., None] * g_l
    dR = (1.0 - w)[..., None] * dY - delta[..., None] * g_r
    dg_l = np.einsum("bht,bhtd->d", delta, O_l)
    dg_r = -np.einsum("bht,bhtd->d", delta, R_tok)
    return dO, dR, dg_l, dg_r


def local_attention_backward(q, k, v, O, LSE, dO, lay: SeqLayout, qblk: int = 256):
    """Backward of :func:`local_attention` (flash-style, recomputing P from LSE).

    D_i = dO_i.O_i;  dS_ij = P_ij (dO_i.v_j - D_i) / sqrt(Dh);
    dq_i = sum_j dS_ij k_j;  dk_j = sum_i dS_ij q_i;  dv_j = sum_i P_ij dO_i.
    """
    B, H, T, Dh = q.shape
    scale = 1.0 / math.sqrt(Dh)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    Dsum = np.einsum("bhtd,bhtd->bht", dO, O)
    for a in range(0, T, qblk):
        b = min(a + qblk, T)
        ka = int(lay.key_lo[a:b].min())
        kb = int(lay.key_hi[a:b].max()) + 1
        if kb <= ka:
            continue
        j = np.arange(ka, kb)
        allowed = (j[None, :] >= lay.key_lo[a:b, None]) & (j[None, :] <= lay.key_hi[a:b, None])
        s = np.einsum("bhid,bhjd->bhij", q[:, :, a:b], k[:, :, ka:kb]) * scale
        lse = LSE[:, :, a:b, None]
        P = np.where(allowed & np.isfinite(lse), np.exp(s - np.where(np.isfinite(lse), lse, 0.0)), 0.0)
        dP = np.einsum("bhid,bhjd->bhij", dO[:, :, a:b], v[:, :, ka:kb])
        dS = P * (dP - Dsum[:, :, a:b, None]) * scale
        dq[:, :, a:b] += np.einsum("bhij,bhjd->bhid", dS, k[:, :, ka:kb])
        dk[:, :, ka:kb] += np.einsum("bhij,bhid->bhjd", dS, q[:, :, a:b])
        dv[:, :, ka:kb] += np.einsum("bhij,bhid->bhjd", P, dO[:, :, a:b])
    return dq, dk, dv


def latent_attention_backward(rq, gk, gv, L, P, dL):
    """Backward of :func:`latent_attention` given its weights P.

    D_s = dL_s.L_s;  dS_sn = P_sn (dL_s.gv_n - D_s) / sqrt(Ldh);
    drq_s = sum_n dS_sn gk_n;  dgk_n = sum_s dS_sn rq_s;  dgv_n = sum_s P_sn dL_s.
    """
    Ldh = rq.shape[-1]
    scale = 1.0 / math.sqrt(Ldh)
    Dsum = np.einsum("bhsd,bhsd->bhs", dL, L)
    dP = np.einsum("bhsd,bhnd->bhsn", dL, gv)
    dS = P * (dP - Dsum[..., None]) * scale
    drq = np.einsum("bhsn,bhnd->bhsd", dS, gk)
    dgk = np.einsum("bhsn,bhsd->bhnd", dS, rq)
    dgv = np.einsum("bhsn,bhsd->bhnd", P, dL)
    return drq, dgk, dgv


def module_backward(params: dict, x: np.ndarray, shape: BlockShape, cache: dict, dout: np.ndarray):
    """Gradients of sum(out * dout) w.r.t. x and every parameter.

    Returns ``(dx, grads)`` where grads maps :data:`PARAM_NAMES` to arrays.
    """
    B, T, D = x.shape
    H, Dh = shape.n_heads, shape.head_dim
    Lh, Ldh, Ld = shape.latent_heads, shape.latent_head_dim, shape.latent_d_model
    lay: SeqLayout = cache["lay"]
    g = {}

    # out projection
    g["out.weight"] = np.einsum("btk,btd->kd", dout, cache["Y_flat"])
    g["out.bias"] = dout.sum(axis=(0, 1))
    dY = (dout @ params["out.weight"]).reshape(B, T, H, Dh).transpose(0, 2, 1, 3)

    # gate
    dO_l, dR_tok, dg_l, dg_r = gate_backward(dY, cache["O_l"], cache["R_tok"], cache["w"],
                                             params["gate_local.weight"][0], params["gate_remote.weight"][0])
    g["gate_local.weight"] = dg_l[None, :]
    g["gate_remote.weight"] = dg_r[None, :]

    # remote: per-token grads folded onto the latent queries, then r_out
    dR_tok_flat = dR_tok.transpose(0, 2, 1, 3).reshape(B, T, D)
    dR_q = np.zeros((B, lay.n_q, D))
    np.add.at(dR_q, (slice(None), cache["tok_q"]), dR_tok_flat)
    g["r_out.weight"] = np.einsum("bsk,bsl->kl", dR_q, cache["L_flat"])
    g["r_out.bias"] = dR_q.sum(axis=(0, 1))
    dL = (dR_q @ params["r_out.weight"]).reshape(B, lay.n_q, Lh, Ldh).transpose(0, 2, 1, 3)

    drq, dgk, dgv = latent_attention_backward(cache["rq"], cache["gk"], cache["gv"], cache["L"], cache["P"], dL)
    drq_flat = drq.transpose(0, 2, 1, 3).reshape(B, lay.n_q, Ld)
    g["rq_proj.weight"] = np.einsum("bsl,bsd->ld", drq_flat, cache["qsrc"])
    g["rq_proj.bias"] = drq_flat.sum(axis=(0, 1))
    dqsrc = drq_flat @ params["rq_proj.weight"]

    dgkgv = np.stack([dgk.transpose(0, 2, 1, 3), dgv.transpose(0, 2, 1, 3)], axis=2).reshape(B, lay.n_chunks, 2 * Ld)
    g["rkv_proj.weight"] = np.einsum("bnl,bnd->ld", dgkgv, cache["pooled"])
    g["rkv_proj.bias"] = dgkgv.sum(axis=(0, 1))
    dpooled = dgkgv @ params["rkv_proj.weight"]

    dq, dk, dv = local_attention_backward(cache["q"], cache["k"], cache["v"], cache["O_l"], cache["LSE"], dO_l, lay)
    dqkv = np.stack([t.transpose(0, 2, 1, 3) for t in (dq, dk, dv)], axis=2).reshape(B, T, 3 * D)
    g["qkv_proj.weight"] = np.einsum("btk,btd->kd", dqkv, x)
    g["qkv_proj.bias"] = dqkv.sum(axis=(0, 1))

    dx = dqkv @ params["qkv_proj.weight"]
    counts = np.array([min((n + 1) * lay.chunk, T) - n * lay.chunk for n in range(lay.n_chunks)], dtype=np.float64)
    dx += (dpooled / counts[None, :, None])[:, lay.chunk_ids]
    if shape.macro:
        dx += dqsrc[:, np.arange(T) // lay.qb] / lay.qb
    else:
        dx += dqsrc
    return dx, g


def init_params(shape: BlockShape, rng: np.random.Generator, std: float = 0.02,
                n_layers: int | None = None) -> dict:
    """Parameters drawn like ``LocalLatentLM._init_weights`` (models.py:520-546):
    N(0, std) weights, zero biases, ``out``/``r_out`` scaled by 1/sqrt(2 n_layers)
    when ``n_layers`` is given.  Biases are drawn non-zero when ``n_layers`` is
    None so tests exercise them."""
    p = {}
    for name, shp in param_shapes(shape).items():
        if name.endswith(".bias"):
            p[name] = np.zeros(shp) if n_layers is not None else rng.normal(0.0, std, size=shp)
        else:
            p[name] = rng.normal(0.0, std, size=shp)
            if n_layers is not None and name.split(".")[0] in ("out", "r_out"):
                p[name] = p[name] / math.sqrt(2 * n_layers)
    return p


def cross_entropy_rows(logits: np.ndarray, targets: np.ndarray, ignore_index: int = -100):
    """Per-row cross entropy of the LM head (reference train.py:354-357, ``F.cross_entropy`` over
    ``[rows, V]`` logits with its default ``ignore_index=-100`` and mean reduction; :358 ``argmax``):
    returns float64 ``loss [rows]`` (``logsumexp(x) - x[t]``, 0 for ignored rows), ``pred [rows]``
    (first index of the maximum, as torch's argmax) and ``grad [rows, V]`` = ``softmax(x) - onehot(t)``
    (0 for ignored rows) -- the gradient of the summed loss; the mean's gradient divides it by the
    number of rows that count."""
    x = np.asarray(logits, dtype=np.float64)
    t = np.asarray(targets).reshape(-1).astype(np.int64)
    m = x.max(axis=1, keepdims=True)
    e = np.exp(x - m)
    s = e.sum(axis=1, keepdims=True)
    lse = (m + np.log(s))[:, 0]
    keep = t != ignore_index
    tt = np.where(keep, t, 0)
    loss = np.where(keep, lse - x[np.arange(x.shape[0]), tt], 0.0)
    grad = e / s
    grad[np.arange(x.shape[0]), tt] -= 1.0
    grad[~keep] = 0.0
    return loss, x.argmax(axis=1), grad
