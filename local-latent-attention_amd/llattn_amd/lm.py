"""The language model around the attention block, for full training steps with the HIP block in every layer.

Module tree, parameter names, initialisation and forward follow the
reference LM (reference models.py:40-58 ``RMSNorm`` / ``FeedForward``,
:490-502 ``TransformerBlock``, :505-580 ``LocalLatentLM``), so its state
dicts load here and the other way round.  The attention of every block is
:func:`~llattn_amd.config.build_attention` (the gfx950 HIP block), as the
reference builds it when ``use_triton_kernel`` is set (reference
models.py:465-488), and the norms run on the gfx950 RMSNorm kernels
(:func:`~llattn_amd.norm.rms_norm`, bf16 output under autocast).
``attention_factory`` / ``norm_factory`` replace them, e.g. with other
implementations to compare against.

:func:`lm_loss` is the token-level loss and metrics of the reference trainer
(reference train.py:340-370, ``compute_loss_and_metrics`` for [B, T] targets);
:meth:`LocalLatentLM.loss` computes the same from the hidden states with the
head and the cross entropy in row chunks (no full logits tensor),
:func:`make_optimizer` its AdamW set-up (reference train.py:851-859) and
:func:`train_step` one optimiser step as its loop runs it (reference
train.py:960-1037, one micro-step, gradient clipping, no loss scaling in bf16).
"""
from __future__ import annotations

import math
from typing import Callable, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

from .config import MODEL_PRESETS, ModelConfig, build_attention
from .norm import add_rms_norm, rms_norm


class RMSNorm(nn.Module):
    """reference models.py:40-47 (same parameter and eps), on the gfx950 kernels."""

    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rms_norm(x, self.weight, self.eps)


class FeedForward(nn.Module):
    """reference models.py:50-58 (``w2(gelu(w1 x))``; dropout 0 is the identity).  Under bf16 autocast on the
    GPU it runs as :func:`llattn_amd.ffn.feed_forward` (the GELU in the GEMM epilogues)."""

    def __init__(self, config: ModelConfig) -> None:
        super().__init__()
        self.w1 = nn.Linear(config.d_model, config.d_ff)
        self.w2 = nn.Linear(config.d_ff, config.d_model)
        self.dropout = nn.Dropout(config.dropout)
        self.fused = True  # False: the reference's separate torch ops (a comparison model sets it)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # bf16 autocast on the GPU without active dropout: both products on the MFMA GEMM, GELU in their epilogues
        if (self.fused and x.is_cuda and torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16
                and (self.dropout.p == 0.0 or not self.training)):
            from .ffn import feed_forward
            return feed_forward(x, self.w1, self.w2)
        return self.dropout(self.w2(F.gelu(self.w1(x))))


class TransformerBlock(nn.Module):
    """Pre-norm residual block (reference models.py:490-502)."""

    def __init__(self, config: ModelConfig, attention_factory: Callable[[ModelConfig], nn.Module],
                 norm_factory: Callable[[int], nn.Module] = RMSNorm) -> None:
        super().__init__()
        self.norm1 = norm_factory(config.d_model)
        self.norm2 = norm_factory(config.d_model)
        self.attn = attention_factory(config)
        self.ff = FeedForward(config)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.norm1(x))
        return x + self.ff(self.norm2(x))


class LocalLatentLM(nn.Module):
    """Token + learned position embeddings, ``n_layers`` blocks, final norm, LM head tied to the token
    embedding (reference models.py:505-580)."""

    def __init__(self, config: ModelConfig, attention_factory: Optional[Callable[[ModelConfig], nn.Module]] = None,
                 norm_factory: Optional[Callable[[int], nn.Module]] = None) -> None:
        super().__init__()
        self.config = config
        self.checkpoint_blocks = config.checkpoint_blocks
        self.fuse_residual_norms = True  # residual adds inside the next norm (same values, fewer passes)
        factory = attention_factory or build_attention
        norm = norm_factory or RMSNorm
        self.embedding = nn.Embedding(config.vocab_size, config.d_model)
        self.position = nn.Embedding(config.max_seq_len, config.d_model)
        self.blocks = nn.ModuleList([TransformerBlock(config, factory, norm) for _ in range(config.n_layers)])
        self.norm = norm(config.d_model)
        self.lm_head = nn.Linear(config.d_model, config.vocab_size, bias=False)
        self.lm_head.weight = self.embedding.weight
        self._init_weights(config.n_layers)

    def _init_weights(self, n_layers: int) -> None:
        """N(0, 0.02) for every Linear and Embedding, zero biases, the residual output projections
        (``out``, ``r_out``, ``w2``) scaled by 1/sqrt(2 n_layers); the tied head is skipped (reference
        models.py:520-546).  The gate vectors are Linear layers too, so they get N(0, 0.02)."""
        output_projs = {"out", "r_out", "w2"}
        for name, module in self.named_modules():
            if module is self.lm_head:
                continue
            if isinstance(module, nn.Linear):
                nn.init.normal_(module.weight, mean=0.0, std=0.02)
                if module.bias is not None:
                    nn.init.zeros_(module.bias)
                if name.rsplit(".", 1)[-1] in output_projs:
                    module.weight.data.mul_(1.0 / math.sqrt(2 * n_layers))
            elif isinstance(module, nn.Embedding):
                nn.init.normal_(module.weight, mean=0.0, std=0.02)

    # profiling API of the reference LM (reference models.py:548-565): per-block stats averaged
    def set_profile(self, enabled: bool) -> None:
        for block in self.blocks:
            block.attn.set_profile(enabled)

    def get_profile_stats(self) -> dict[str, float]:
        totals: dict[str, float] = {}
        count = 0
        for block in self.blocks:
            stats = block.attn.get_profile_stats()
            if not stats:
                continue
            count += 1
            for k, v in stats.items():
                totals[k] = totals.get(k, 0.0) + v
        return {k: v / count for k, v in totals.items()} if count else {}

    def hidden(self, input_ids: torch.Tensor) -> torch.Tensor:
        """The final-norm hidden states ``[B, T, D]`` that the tied head maps to logits."""
        _, seq_len = input_ids.shape
        pos = torch.arange(seq_len, device=input_ids.device)
        x = self.embedding(input_ids) + self.position(pos).unsqueeze(0)
        if self._fused_norms(x):
            return self._hidden_fused(x)
        for block in self.blocks:
            if self.checkpoint_blocks and self.training:
                x = checkpoint(block, x, use_reentrant=False)
            else:
                x = block(x)
        return self.norm(x)

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        return self.lm_head(self.hidden(input_ids))

    @torch.no_grad()
    def next_token_logits(self, context: torch.Tensor) -> torch.Tensor:
        """Logits ``[B, V]`` of the last position of each context row: the full forward over the context, which
        reference generate.py:188-190 re-runs for every new token (the latent chunk and the local block depend
        on the context length, so no earlier state can be reused), with the tied head applied to the last
        position only and nothing kept for a backward."""
        return self.lm_head(self.hidden(context)[:, -1])

    @torch.no_grad()
    def generate(self, prompt_ids: torch.Tensor, max_new_tokens: int, temperature: float = 0.0, top_k: int = 0,
                 eos_token_id: Optional[int] = None, generator: Optional[torch.Generator] = None) -> torch.Tensor:
        """Continue ``prompt_ids [1, P]`` by up to ``max_new_tokens`` tokens, one full re-forward of the last
        ``max_seq_len`` tokens per new token (reference generate.py:169-204).  ``temperature`` 0 takes the
        argmax, otherwise the token is drawn from softmax(logits / temperature), restricted to the ``top_k``
        largest logits when ``top_k`` > 0.  Stops after ``eos_token_id``.  The reference sampler's repetition
        penalty and n-gram bans (generation UX) are not part of this.  Returns ``[1, P + n]``."""
        if prompt_ids.dim() != 2 or prompt_ids.shape[0] != 1 or prompt_ids.shape[1] == 0:
            raise ValueError("prompt_ids must be a non-empty [1, P] tensor")
        ids = prompt_ids
        for _ in range(max_new_tokens):
            logits = self.next_token_logits(ids[:, -self.config.max_seq_len:]).float()
            if temperature <= 0.0:
                nxt = logits.argmax(-1, keepdim=True)
            else:
                logits = logits / temperature
                if top_k > 0:
                    kth = torch.topk(logits, min(top_k, logits.shape[-1]), dim=-1).values[:, -1:]
                    logits = logits.masked_fill(logits < kth, float("-inf"))
                nxt = torch.multinomial(torch.softmax(logits, -1), 1, generator=generator)
            ids = torch.cat([ids, nxt.to(ids.dtype)], dim=1)
            if eos_token_id is not None and int(nxt) == eos_token_id:
                break
        return ids

    def _fused_norms(self, x: torch.Tensor) -> bool:
        """Whether each residual add runs inside the following norm (:func:`~llattn_amd.norm.add_rms_norm`): all
        norms are this module's GPU RMSNorm, the stream is fp32 and blocks are not checkpointed one by one."""
        if not self.fuse_residual_norms or not len(self.blocks) or (self.checkpoint_blocks and self.training):
            return False
        norms = [self.norm] + [m for b in self.blocks for m in (b.norm1, b.norm2)]
        return x.is_cuda and x.dtype == torch.float32 and all(type(n) is RMSNorm for n in norms)

    def _hidden_fused(self, x: torch.Tensor) -> torch.Tensor:
        # x_{i+1} = x_i + attn(norm1(x_i)) + ff(norm2(...)) as in TransformerBlock.forward, with each sum formed by
        # the norm that reads it: norm2 of the same block, then norm1 of the next block (the final norm last)
        blocks = list(self.blocks)
        h = blocks[0].norm1(x)
        for i, blk in enumerate(blocks):
            x, h2 = add_rms_norm(x, blk.attn(h), blk.norm2.weight, blk.norm2.eps)
            nxt = blocks[i + 1].norm1 if i + 1 < len(blocks) else self.norm
            x, h = add_rms_norm(x, blk.ff(h2), nxt.weight, nxt.eps)
        return h

    def loss(self, input_ids: torch.Tensor, targets: torch.Tensor, chunk_rows: int = 8192):
        """:func:`lm_loss` of ``self(input_ids)`` without the ``[B*T, V]`` logits: the tied head and the cross
        entropy run in row chunks on the gfx950 kernels (:func:`~llattn_amd.xent.lm_head_loss`)."""
        from .xent import head_supported, lm_head_loss
        V, D = self.lm_head.weight.shape
        if not head_supported(V, D):  # vocabularies the chunked kernels do not take: full logits, as the reference
            return lm_loss(self.lm_head(self.hidden(input_ids)), targets)
        loss, pred = lm_head_loss(self.hidden(input_ids), self.lm_head.weight, targets, chunk_rows=chunk_rows)
        return loss, _metrics(loss, (pred == targets).float().mean())


def build_model(preset: Optional[str] = None, attention_factory=None, norm_factory=None,
                **overrides) -> LocalLatentLM:
    """``LocalLatentLM`` from ``ModelConfig`` defaults, a trainer preset's architecture keys (reference
    train.py:71-102) and explicit overrides, in that order of precedence (lowest first)."""
    fields = dict(MODEL_PRESETS[preset]) if preset else {}
    fields.update(overrides)
    return LocalLatentLM(ModelConfig(**fields), attention_factory, norm_factory)


def lm_loss(logits: torch.Tensor, targets: torch.Tensor):
    """Mean next-token cross entropy over ``[B, T]`` targets and the trainer's metric tensors (no host
    synchronisation), as reference train.py:354-370 computes them."""
    flat = logits.reshape(-1, logits.size(-1))
    loss = F.cross_entropy(flat, targets.reshape(-1))
    return loss, _metrics(loss, (logits.argmax(dim=-1) == targets).float().mean())


def _metrics(loss: torch.Tensor, acc: torch.Tensor) -> dict:
    loss_det = loss.detach()
    return {"eval_loss": loss_det, "eval_acc": acc, "eval_perplexity": torch.exp(torch.clamp(loss_det, max=20.0)),
            "eval_bpt": loss_det / math.log(2.0)}


def make_optimizer(model: nn.Module, lr: float = 3e-4) -> torch.optim.Optimizer:
    """AdamW with weight decay 0.1 on matrices and 0 on vectors, betas (0.9, 0.95), fused on GPU (reference
    train.py:851-859; default lr of reference train.py:159)."""
    decay = [p for p in model.parameters() if p.ndim >= 2]
    no_decay = [p for p in model.parameters() if p.ndim < 2]
    fused = next(model.parameters()).device.type == "cuda"
    return torch.optim.AdamW([{"params": decay, "weight_decay": 0.1}, {"params": no_decay, "weight_decay": 0.0}],
                             lr=lr, betas=(0.9, 0.95), fused=fused)


def train_step(model: nn.Module, optimizer: torch.optim.Optimizer, inputs: torch.Tensor, targets: torch.Tensor,
               grad_clip: float = 1.0, fused_loss: bool = True) -> torch.Tensor:
    """One bf16-autocast optimiser step: forward, loss, backward, gradient clipping, AdamW update, gradients
    cleared (reference train.py:960-1037 with one micro-step).  ``fused_loss``: the chunked head + cross entropy
    (:meth:`LocalLatentLM.loss`) instead of full logits and ``F.cross_entropy``.  Returns the detached loss (no
    sync)."""
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        if fused_loss:
            loss, _ = model.loss(inputs, targets)
        else:
            loss, _ = lm_loss(model(inputs), targets)
        loss.backward()
    if grad_clip > 0:
        torch.nn.utils.clip_grad_norm_(model.parameters(), grad_clip)
    optimizer.step()
    optimizer.zero_grad(set_to_none=True)
    return loss.detach()
