"""Drop-in attention block backed by the gfx950 HIP kernels.

``LocalLatentAttentionTriton`` keeps the constructor, ``forward`` and profiling
surface of the reference's fused module (reference llattn_triton.py:33-176) and
the parameter names, shapes, initialisation order and math of the reference
PyTorch block ``LocalLatentAttention`` (reference models.py:61-462), so
checkpoints interchange with the PyTorch path and outputs match it.

Data flow of one forward (B, T, D = batch, tokens, d_model):

1. ``qkvr = x @ [W_qkv; W_rq]^T + b`` -- one GEMM for q|k|v and the token-wise
   latent queries (macro-block mode: ``qkv`` GEMM, HIP query-block pooling,
   ``rq_proj`` GEMM); under bf16 autocast through :func:`~llattn_amd.linear.project`,
   whose weight gradients come from the gfx950 MFMA kernel in fp32, with q|k|v stored
   split-head (``[B][3H][T][Dh]`` slabs, the latent queries packed after them) so that
   the local-attention kernels stream each head as one contiguous run;
2. ``pooled = chunk means of x`` (HIP) and ``gkgv = rkv_proj(pooled)`` (GEMM);
3. :class:`~llattn_amd.ops.LLAttnCore` -- HIP latent attention, ``r_out``
   GEMM, HIP windowed attention with the gate mix fused in its epilogue;
4. ``out`` GEMM.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from . import _lib as L
from .linear import pack_params, project, project_f32
from .ops import LLAttnCore, _Prof, grad_heads_ok, heads_layout_ok, pool


class LocalLatentAttentionTriton(nn.Module):
    """``LocalLatentAttentionTriton(d_model, n_heads, latent_heads, latent_dim, n_latents, window,
    bias=True, local_block_size=256, latent_query_block_size=0)``.

    The first six arguments are those the reference dispatcher passes
    (reference models.py:480-487).  ``local_block_size`` and
    ``latent_query_block_size`` default to the reference ``ModelConfig`` values
    (reference models.py:31, 35).  ``bias`` defaults to True so the parameter set
    equals ``LocalLatentAttention``'s (reference models.py:80-84).
    """

    def __init__(self, d_model: int, n_heads: int, latent_heads: int, latent_dim: int, n_latents: int,
                 window: int, bias: bool = True, local_block_size: int = 256,
                 latent_query_block_size: int = 0) -> None:
        super().__init__()
        # reference llattn_triton.py:45-47 and models.py:64-65
        assert d_model % n_heads == 0, "d_model must be divisible by n_heads"
        assert latent_dim % latent_heads == 0, "latent_dim must be divisible by latent_heads"
        self.d_model = d_model
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        self.latent_heads = latent_heads
        self.latent_dim = latent_dim
        self.latent_d_model = latent_dim
        self.latent_head_dim = latent_dim // latent_heads
        self.n_latents = n_latents
        self.latent_tokens = n_latents
        self.window = window
        self.local_block_size = local_block_size
        self.latent_query_block_size = max(0, latent_query_block_size)
        # same names, shapes and creation order as reference models.py:80-90
        self.qkv_proj = nn.Linear(d_model, 3 * d_model, bias=bias)
        self.rq_proj = nn.Linear(d_model, latent_dim, bias=bias)
        self.rkv_proj = nn.Linear(d_model, 2 * latent_dim, bias=bias)
        self.r_out = nn.Linear(latent_dim, d_model, bias=bias)
        self.out = nn.Linear(d_model, d_model, bias=bias)
        self.gate_local = nn.Linear(self.head_dim, 1, bias=False)
        self.gate_remote = nn.Linear(self.head_dim, 1, bias=False)
        self.profile_enabled = False
        self.profile_totals: dict[str, float] = {}
        self.profile_steps = 0

    # ---- checkpoint compatibility: split legacy projections (reference models.py:98-129)
    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                              error_msgs):
        for fused, parts in (("qkv_proj", ("q_proj", "k_proj", "v_proj")), ("rkv_proj", ("rk_proj", "rv_proj"))):
            for kind in ("weight", "bias"):
                key = f"{prefix}{fused}.{kind}"
                old = [f"{prefix}{p}.{kind}" for p in parts]
                if key not in state_dict and all(o in state_dict for o in old):
                    state_dict[key] = torch.cat([state_dict.pop(o) for o in old], dim=0)
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                                      error_msgs)

    # ---- profiling API (reference models.py:131-152; llattn_triton.py:83-90)
    def set_profile(self, enabled: bool) -> None:
        self.profile_enabled = enabled
        self.profile_totals = {}
        self.profile_steps = 0

    def get_profile_stats(self) -> dict[str, float]:
        if not self.profile_enabled or self.profile_steps == 0:
            return {}
        n = self.profile_steps
        return {f"profile_{k}": v / n for k, v in self.profile_totals.items()}

    def layout(self, B: int, T: int) -> L.Layout:
        return L.resolve_layout(B, T, self.d_model, self.n_heads, self.latent_dim, self.latent_heads, self.window,
                                self.local_block_size, self.n_latents, self.latent_query_block_size)

    def forward(self, x: torch.Tensor, _positions: Optional[torch.Tensor] = None) -> torch.Tensor:
        B, T, D = x.shape
        if D != self.d_model:
            raise ValueError(f"expected d_model={self.d_model}, got input of width {D}")
        L.require_gpu(x)
        lay = self.layout(B, T)
        prof = _Prof(self.profile_enabled, x.device) if self.profile_enabled else None
        if prof is not None:
            prof.start()
        macro = self.latent_query_block_size > 1
        # bf16 autocast (the reference trainer's mode): projections in bf16 with fp32 weight gradients
        bf16 = torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16
        latents = (lay.chunk, lay.n_chunks, L.DIV_COUNT)
        pooled = None
        packed = self._packed_weights(macro) if bf16 else {}
        # bf16: q|k|v (and token-wise latent queries) stored split-head -- each head of a sequence one contiguous
        # run for the attention kernels, written and read in that order by the projection's GEMMs
        heads = bf16 and heads_layout_ok(lay, D, not macro)
        hl = (T, lay.Dh, 3 * self.n_heads, 0 if macro else lay.Ldh) if heads else None
        if macro and bf16:
            # both poolings of x ride on the projection, whose backward adds their gradients in place
            qkvr, pq, pooled = project(x, self.qkv_proj, pools=[(lay.q_block, lay.n_q, L.DIV_SEG), latents],
                                       packed=packed["qkv"], heads=hl)
            rq = project(pq, self.rq_proj, packed=packed["rq"])
        elif macro:
            qkvr = project_f32(x, self.qkv_proj)
            rq = project_f32(pool(x, lay.q_block, lay.n_q, L.DIV_SEG), self.rq_proj)
        elif bf16:
            qkvr, pooled = project(x, self.qkv_proj, self.rq_proj, pools=[latents], packed=packed["qkv"], heads=hl)
            rq = None
        else:
            qkvr = project_f32(x, self.qkv_proj, self.rq_proj)
            rq = None
        if prof is not None:
            prof.lap("qkv_ms")
        if pooled is None:
            pooled = pool(x, *latents)
        # the pooled latents' projection (256 rows at config 2) on the MFMA GEMM as well: split-K forward,
        # bias gradient from the weight-gradient pass
        gkgv = project(pooled, self.rkv_proj, packed=packed["rkv"]) if bf16 else project_f32(pooled, self.rkv_proj)
        if prof is not None:
            prof.lap("pool_ms")
        rqc = None if rq is None else rq.to(qkvr.dtype)
        # forward only (no_grad, e.g. generation): the kernels skip what only the backward reads
        saved = torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))
        # bf16: the output projection's input gradient comes back as [B][H][T][Dh] slabs for the local backward
        dy_heads = bf16 and grad_heads_ok(B * T, self.d_model, D, lay.Dh)
        y = LLAttnCore.apply(qkvr, rqc, gkgv.to(qkvr.dtype), self.gate_local.weight, self.gate_remote.weight,
                             self.r_out.weight, self.r_out.bias, lay, prof, packed.get("r_out"), saved, heads,
                             dy_heads)
        if prof is not None:
            # the gate mix runs in the local kernel's epilogue: its time is in local_attention_ms
            prof.t["gate_mix_ms"] = 0.0
            self._record_profile(prof, lay)
        if not bf16:
            return project_f32(y, self.out)
        return project(y, self.out, packed=packed["out"], grad_heads=(T, lay.Dh, self.n_heads) if dy_heads else None)

    def _packed_weights(self, macro: bool) -> dict:
        """The bf16 copies of every projection weight that this forward multiplies with (what bf16 autocast casts
        per forward), the concatenated fp32 biases of qkv_proj + rq_proj, and bf16 W^T copies of the qkv|rq,
        out and r_out weights for their input gradients, written by one llattn_cast_transposed launch.  Single
        projections take their fp32 bias as it is."""
        qkv = [self.qkv_proj] if macro else [self.qkv_proj, self.rq_proj]
        has_b = self.qkv_proj.bias is not None
        # the weights whose input gradients have token-count rows also get their W^T copy from the same launch
        groups = [([m.weight for m in qkv], torch.bfloat16, True)]
        if has_b:
            groups.append(([m.bias for m in qkv], torch.float32))
        singles = (["rq"] if macro else []) + ["rkv", "out", "r_out"]
        mods = {"rq": self.rq_proj, "rkv": self.rkv_proj, "out": self.out, "r_out": self.r_out}
        groups += [([mods[k].weight], torch.bfloat16, k in ("out", "r_out")) for k in singles]
        outs = pack_params(groups)
        w, w_t = outs[0]
        packed = {"qkv": (w, outs[1] if has_b else None, w_t)}
        for i, k in enumerate(singles):
            o = outs[(2 if has_b else 1) + i]
            if k == "r_out":
                packed[k] = o  # (W, W^T)
            elif k == "out":
                packed[k] = (o[0], mods[k].bias, o[1])
            else:
                packed[k] = (o, mods[k].bias)
        return packed

    def _record_profile(self, prof, lay: L.Layout) -> None:
        t = prof.t
        tot = self.profile_totals
        total = sum(t.values())
        for key in ("qkv_ms", "pool_ms", "local_attention_ms", "latent_attention_ms", "gate_mix_ms"):
            tot[key] = tot.get(key, 0.0) + t.get(key, 0.0)
        tot["local_latent_total_ms"] = tot.get("local_latent_total_ms", 0.0) + total
        tot["gate_mean"] = tot.get("gate_mean", 0.0) + float(prof.gate_mean.mean().item())
        tot["seq_len"] = tot.get("seq_len", 0.0) + lay.T
        tot["local_block_size"] = tot.get("local_block_size", 0.0) + lay.block
        tot["latent_count"] = tot.get("latent_count", 0.0) + lay.n_chunks
        tot["latent_chunk_size"] = tot.get("latent_chunk_size", 0.0) + lay.chunk
        tot["latent_query_block_size"] = tot.get("latent_query_block_size", 0.0) + lay.q_block
        self.profile_steps += 1


# name used by this package; the class above keeps the reference module's name
LocalLatentAttentionHIP = LocalLatentAttentionTriton
