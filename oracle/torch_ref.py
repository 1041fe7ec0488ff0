"""PyTorch CPU restatement of the reference block (TEST INFRASTRUCTURE ONLY).

Same semantics as ``oracle/llattn_oracle.py`` (the reference PyTorch path,
``/root/reference/models.py:61-462``) written with differentiable torch ops
so autograd supplies the backward.  It is faster than the float64 numpy
oracle at the large shapes (multithreaded fp32 GEMMs, query-blocked local
attention as in models.py:251-276), so it serves as

* the fp32 reference for GPU parity checks at BASELINE sizes, and
* ``bench.py``'s ``cpu_baseline`` leg: the reference PyTorch CPU path,
  timed on the host cores.

Pinned by ``tests/test_oracle_torch.py`` against the reference golden vectors
and the numpy oracle.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` may import it.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .llattn_oracle import BlockShape, seq_layout


def _masked_softmax(s: torch.Tensor, allowed: torch.Tensor) -> torch.Tensor:
    """Softmax over the last dim restricted to ``allowed``; rows with no allowed entry give 0."""
    s = s.masked_fill(~allowed, float("-inf"))
    has = allowed.any(dim=-1, keepdim=True)
    s = torch.where(has, s, torch.zeros_like(s))
    return torch.softmax(s, dim=-1) * has


def local_attention(q, k, v, shape: BlockShape, T: int) -> torch.Tensor:
    """q, k, v: [B, H, T, Dh] -> [B, H, T, Dh] (reference models.py:232-305)."""
    lay = seq_layout(shape, T)
    lo = torch.from_numpy(lay.key_lo)
    hi = torch.from_numpy(lay.key_hi)
    scale = 1.0 / math.sqrt(q.shape[-1])
    outs = []
    for a in range(0, T, lay.bs):
        b = min(a + lay.bs, T)
        ka = max(0, a - shape.window)
        kb = b
        j = torch.arange(ka, kb)
        allowed = (j[None, :] >= lo[a:b, None]) & (j[None, :] <= hi[a:b, None])
        s = torch.matmul(q[:, :, a:b], k[:, :, ka:kb].transpose(-1, -2)) * scale
        outs.append(torch.matmul(_masked_softmax(s, allowed), v[:, :, ka:kb]))
    return torch.cat(outs, dim=2)


def block_forward(params: dict, x: torch.Tensor, shape: BlockShape) -> torch.Tensor:
    """Forward of ``LocalLatentAttention`` (reference models.py:307-462); differentiable."""
    B, T, D = x.shape
    H, Dh = shape.n_heads, shape.head_dim
    Lh, Ldh, Ld = shape.latent_heads, shape.latent_head_dim, shape.latent_d_model
    lay = seq_layout(shape, T)

    qkv = F.linear(x, params["qkv_proj.weight"], params["qkv_proj.bias"]).view(B, T, 3, H, Dh)
    q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))

    # chunk means over real tokens
    seg = torch.from_numpy(lay.chunk_ids)
    counts = torch.bincount(seg, minlength=lay.n_chunks).to(x.dtype)
    pooled = torch.zeros(B, lay.n_chunks, D, dtype=x.dtype).index_add(1, seg, x) / counts[None, :, None]
    gkgv = F.linear(pooled, params["rkv_proj.weight"], params["rkv_proj.bias"]).view(B, lay.n_chunks, 2, Lh, Ldh)
    gk, gv = gkgv[:, :, 0].transpose(1, 2), gkgv[:, :, 1].transpose(1, 2)
    if shape.macro:
        blk = torch.arange(T) // lay.qb
        qsrc = torch.zeros(B, lay.n_q, D, dtype=x.dtype).index_add(1, blk, x) / lay.qb
    else:
        qsrc = x
    rq = F.linear(qsrc, params["rq_proj.weight"], params["rq_proj.bias"]).view(B, lay.n_q, Lh, Ldh).transpose(1, 2)

    local = local_attention(q, k, v, shape, T)

    n = torch.arange(lay.n_chunks)
    allowed = n[None, :] < torch.from_numpy(lay.q_chunk_ids)[:, None]
    lat = torch.matmul(_masked_softmax(torch.matmul(rq, gk.transpose(-1, -2)) / math.sqrt(Ldh), allowed), gv)
    remote = F.linear(lat.transpose(1, 2).reshape(B, lay.n_q, Ld), params["r_out.weight"], params["r_out.bias"])
    if shape.macro:
        remote = remote[:, torch.arange(T) // lay.qb]
    remote = remote.view(B, T, H, Dh).transpose(1, 2)

    s_l = torch.matmul(local, params["gate_local.weight"][0])
    s_r = torch.matmul(remote, params["gate_remote.weight"][0])
    w = torch.sigmoid(s_l - s_r).unsqueeze(-1)
    mixed = w * local + (1.0 - w) * remote
    return F.linear(mixed.transpose(1, 2).reshape(B, T, D), params["out.weight"], params["out.bias"])


def block_forward_backward(params: dict, x: torch.Tensor, dout: torch.Tensor, shape: BlockShape):
    """Returns (out, dx, grads) for ``sum(out * dout)``."""
    p = {n: t.detach().clone().requires_grad_(True) for n, t in params.items()}
    xx = x.detach().clone().requires_grad_(True)
    out = block_forward(p, xx, shape)
    out.backward(dout)
    return out.detach(), xx.grad, {n: t.grad for n, t in p.items()}
