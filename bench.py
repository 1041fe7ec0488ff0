"""Benchmark of the fused local+latent attention layer, forward + backward, on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2|c3|c4] [--no-cpu-baseline]

One step = one forward and backward of one ``LocalLatentAttention`` layer
(all projections, pooling, latent and local attention, gate, output
projection; gradients of the input and of every parameter) on synthetic
data that is already resident in HBM, under bf16 autocast with fp32 master
weights (how the reference trainer runs it).  The default workload is
the 0.55b-preset layer at B=16, T=2048.

Prints ONE JSON line.  Besides the driver's fields it carries
``roofline`` (the C-ABI entry point with the most time per step, priced
against bf16 MFMA peak for the projection GEMM and against HBM peak for the
attention kernels; durations measured with HIP events on the launch stream
in a second timed region of K steps, because an event record costs the GPU
about 5 us between kernels and would inflate the step time of the first),
``mfma_frac_module`` (algorithmic module FLOPs / step time / bf16 dense
peak), per-kernel event timings, and ``cpu_baseline`` (the reference
PyTorch path restated in fp32, timed on the host cores on a bounded
sample).  Diagnostics go to stderr.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import torch
import torch.nn as nn
import torch.nn.functional as F

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "local-latent-attention_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK = 2.5e15

CONFIGS = {
    # name: (B, T, d_model, n_heads, window, local_block_size, latent_tokens, latent_d_model, latent_heads, qbs)
    "c2": dict(B=16, T=2048, d_model=1408, n_heads=16, window=64, local_block_size=256, latent_tokens=16,
               latent_d_model=512, latent_heads=8, qbs=0,
               workload="0.55b-preset LocalLatentAttention layer fwd+bwd (BASELINE config 2)"),
    "c3": dict(B=2, T=16384, d_model=1024, n_heads=16, window=512, local_block_size=256, latent_tokens=256,
               latent_d_model=64, latent_heads=2, qbs=0,
               workload="long-context latent-heavy layer fwd+bwd (BASELINE config 3)"),
    "c4": dict(B=4, T=8192, d_model=1024, n_heads=16, window=256, local_block_size=256, latent_tokens=128,
               latent_d_model=64, latent_heads=2, qbs=64,
               workload="macro-block latent query layer fwd+bwd (BASELINE config 4)"),
}


# config 5: the full LM (0.55b preset: reference train.py:73-82; vocab 32000, B16 T2048)
LM_CONFIG = dict(B=16, T=2048, vocab=32000, n_layers=22, d_model=1408, d_ff=4096)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def layout(cfg):
    from llattn_amd import resolve_layout
    return resolve_layout(cfg["B"], cfg["T"], cfg["d_model"], cfg["n_heads"], cfg["latent_d_model"],
                          cfg["latent_heads"], cfg["window"], cfg["local_block_size"], cfg["latent_tokens"],
                          cfg["qbs"])


def key_counts(lay):
    """Exact number of local keys per query (reference models.py:249-292) and visible latents per latent query."""
    import numpy as np
    i = np.arange(lay.T)
    lo = np.maximum(np.maximum(0, i - lay.window), (i // lay.block) * lay.block - lay.window + 1)
    keys = np.maximum(0, i - lo)
    s = np.arange(lay.n_q)
    lat = np.minimum((s * lay.q_block) // lay.chunk, lay.n_chunks)
    return int(keys.sum()), int(lat.sum())


def module_flops(lay):
    """Algorithmic FLOPs of one layer forward + backward: sum of 2*M*N*K over the contractions with exact
    key / latent counts and unpadded head dims; backward = 2 x forward; elementwise work excluded."""
    B, T, H, Dh, Lh, Ldh = lay.B, lay.T, lay.H, lay.Dh, lay.Lh, lay.Ldh
    D, Ld = H * Dh, Lh * Ldh
    nkeys, nlat = key_counts(lay)
    fwd = B * (2 * T * D * 3 * D          # qkv
               + 2 * lay.n_q * D * Ld     # rq
               + 2 * lay.n_chunks * D * 2 * Ld  # rkv
               + 4 * Dh * nkeys * H       # local QK^T and PV
               + 4 * Ldh * nlat * Lh      # latent
               + 2 * lay.n_q * Ld * D     # r_out
               + 2 * T * D * D            # out
               + 4 * Dh * T * H)          # gate dots
    return 3 * fwd


# entry points priced against MFMA peak (their calls state algorithmic FLOPs); the rest against HBM
FLOP_ENTRY_POINTS = ("llattn_gemm",)


def kernel_bytes(lay, es):
    """Algorithmic HBM bytes per launch of each C-ABI entry point (each operand read or written once)."""
    B, T, H, Dh, Lh = lay.B, lay.T, lay.H, lay.Dh, lay.Lh
    D, Ld = H * Dh, lay.Lh * lay.Ldh
    return {
        # q, k, v, y, o_local per token; remote per latent query; lse + w fp32
        "llattn_local_gate_fwd": B * T * (5 * D * es + 8 * H) + B * lay.n_q * D * es,
        # reads q, k, v, o_local, dy, remote, lse, w; writes dq, dk, dv, dremote
        "llattn_local_gate_bwd": B * T * (9 * D * es + 8 * H) + B * lay.n_q * D * es,
        # reads rq, gk, gv; writes latent out + lse
        "llattn_latent_fwd": B * lay.n_q * (2 * Ld * es + 4 * Lh) + B * lay.n_chunks * 2 * Ld * es,
        # reads rq, latent out, dL, lse, gk, gv; writes drq, dgk, dgv
        "llattn_latent_bwd": B * lay.n_q * (4 * Ld * es + 4 * Lh) + B * lay.n_chunks * 4 * Ld * es,
    }


def make_module(cfg, dev):
    from llattn_amd import LocalLatentAttentionTriton
    torch.manual_seed(0)
    m = LocalLatentAttentionTriton(cfg["d_model"], cfg["n_heads"], cfg["latent_heads"], cfg["latent_d_model"],
                                   cfg["latent_tokens"], cfg["window"], local_block_size=cfg["local_block_size"],
                                   latent_query_block_size=cfg["qbs"])
    with torch.no_grad():  # LocalLatentLM init for the 22-layer preset (reference models.py:520-546)
        for name, p in m.named_parameters():
            if name.endswith("bias"):
                p.zero_()
            else:
                p.normal_(0.0, 0.02)
                if name.split(".")[0] in ("out", "r_out"):
                    p.mul_(1.0 / math.sqrt(2 * 22))
    return m.to(dev)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, budget_s: float):
    """The reference PyTorch path (fp32 torch restatement of reference models.py:307-462, autograd backward)
    on the host cores, over the whole workload batch: one warm-up pass, then the median of three timed
    fwd+bwd passes (one when the warm-up alone took more than ``budget_s`` seconds)."""
    from oracle import torch_ref
    from oracle.llattn_oracle import BlockShape
    torch.set_num_threads(os.cpu_count() or 1)
    shape = BlockShape(d_model=cfg["d_model"], n_heads=cfg["n_heads"], window=cfg["window"],
                       local_block_size=cfg["local_block_size"], latent_tokens=cfg["latent_tokens"],
                       latent_d_model=cfg["latent_d_model"], latent_heads=cfg["latent_heads"],
                       latent_query_block_size=cfg["qbs"])
    g = torch.Generator().manual_seed(0)
    D, Ld, Dh = cfg["d_model"], cfg["latent_d_model"], cfg["d_model"] // cfg["n_heads"]
    shapes = {"qkv_proj.weight": (3 * D, D), "qkv_proj.bias": (3 * D,), "rq_proj.weight": (Ld, D),
              "rq_proj.bias": (Ld,), "rkv_proj.weight": (2 * Ld, D), "rkv_proj.bias": (2 * Ld,),
              "r_out.weight": (D, Ld), "r_out.bias": (D,), "out.weight": (D, D), "out.bias": (D,),
              "gate_local.weight": (1, Dh), "gate_remote.weight": (1, Dh)}
    params = {n: torch.randn(s, generator=g) * 0.02 for n, s in shapes.items()}
    B, T = cfg["B"], cfg["T"]
    x = torch.randn(B, T, D, generator=g)
    dout = torch.randn(B, T, D, generator=g)

    def one():
        t0 = time.perf_counter()
        torch_ref.block_forward_backward(params, x, dout, shape)
        return time.perf_counter() - t0

    warm = one()
    runs = sorted(one() for _ in range(3 if warm <= budget_s else 1))
    med = runs[len(runs) // 2]
    return {"value": round(B * T / med, 1), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "cpu_count": os.cpu_count(), "cpu_model": cpu_model(),
            "sample": f"the full workload batch ({B} x {T} tokens), fp32 fwd+bwd of the torch CPU restatement of "
                      f"the reference PyTorch path; 1 warm-up ({warm:.1f} s), median of {len(runs)} timed passes "
                      f"({', '.join(f'{r:.2f}' for r in runs)} s)"}


class TorchPathAttention(nn.Module):
    """The reference's PyTorch attention block (reference models.py:61-462): SDPA per local block with an
    additive float mask (cached per shape), eager latent attention, ``r_out``, the gate softmax and ``out``,
    with the same parameters as the HIP block.  It is the comparison baseline of config 5 (the "PyTorch
    SDPA + eager latent" path on the same GPU) and nothing else."""

    def __init__(self, config):
        super().__init__()
        D, H, Ld = config.d_model, config.n_heads, config.latent_d_model
        self.d_model, self.n_heads, self.head_dim = D, H, D // H
        self.latent_heads, self.latent_head_dim = config.latent_heads, Ld // config.latent_heads
        self.window, self.local_block_size = config.local_window, config.local_block_size
        self.latent_tokens, self.latent_query_block_size = config.latent_tokens, config.latent_query_block_size
        # names, shapes and creation order of reference models.py:80-90
        self.qkv_proj = nn.Linear(D, 3 * D)
        self.rq_proj = nn.Linear(D, Ld)
        self.rkv_proj = nn.Linear(D, 2 * Ld)
        self.r_out = nn.Linear(Ld, D)
        self.out = nn.Linear(D, D)
        self.gate_local = nn.Linear(self.head_dim, 1, bias=False)
        self.gate_remote = nn.Linear(self.head_dim, 1, bias=False)
        self._mask_cache = {}

    def _pool_to_latents(self, x):  # reference models.py:159-214
        B, T, D = x.shape
        chunk = math.ceil(T / min(self.latent_tokens, T))
        full, rem = T // chunk, T % chunk
        parts = [x[:, :full * chunk, :].contiguous().view(B, full, chunk, D).mean(dim=2)] if full else []
        if rem:
            parts.append(x[:, full * chunk:, :].mean(dim=1, keepdim=True))
        pooled = parts[0] if len(parts) == 1 else torch.cat(parts, dim=1)
        ids = (torch.arange(T, device=x.device) // chunk).clamp(max=pooled.size(1) - 1)
        return pooled, ids

    def _pool_query_blocks(self, x, ids):  # reference models.py:216-230
        B, T, D = x.shape
        qb = min(T, self.latent_query_block_size)
        n = math.ceil(T / qb)
        if n * qb > T:
            x = F.pad(x, (0, 0, 0, n * qb - T))
        pooled = x.view(B, n, qb, D).mean(dim=2)
        return pooled, torch.stack([ids[s:min(s + qb, T)].min() for s in range(0, T, qb)])

    def _mask(self, nq, nk, left, device, dtype):  # reference models.py:278-305
        key = (nq, nk, left, device)
        m = self._mask_cache.get(key)
        if m is None:
            dist = (left + torch.arange(nq, device=device)).unsqueeze(1) - torch.arange(nk, device=device)
            allowed = (dist > 0) & (dist <= self.window)
            m = torch.full((nq, nk), float("-inf"), device=device).masked_fill(allowed, 0.0)
            self._mask_cache[key] = m
        return m.to(dtype=dtype)

    @staticmethod
    def _sdpa(q, k, v, mask):
        """SDPA as the reference calls it.  On the GPU in bf16 the fused memory-efficient kernel is required:
        bf16 batched products with a transposed right operand (what SDPA's math path and its backward issue)
        have faulted MI355X boxes under this software stack."""
        if q.is_cuda and q.dtype != torch.float32:
            from torch.nn.attention import SDPBackend, sdpa_kernel
            with sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION]):
                return F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask)

    def _local_attention(self, q, k, v):  # reference models.py:232-276
        B, _, T, _ = q.shape
        bs = min(T, max(self.window, self.local_block_size))
        out = q.new_empty(B, self.n_heads, T, self.head_dim)
        for a in range(0, T, bs):
            b = min(a + bs, T)
            ka = max(0, a - self.window + 1)
            out[:, :, a:b, :] = self._sdpa(q[:, :, a:b, :], k[:, :, ka:b, :], v[:, :, ka:b, :],
                                           self._mask(b - a, b - ka, a - ka, q.device, q.dtype))
        return out

    def forward(self, x):  # reference models.py:307-462
        B, T, D = x.shape
        H, Dh, Lh, Ldh = self.n_heads, self.head_dim, self.latent_heads, self.latent_head_dim
        q, k, v = (t.transpose(1, 2) for t in self.qkv_proj(x).view(B, T, 3, H, Dh).unbind(dim=2))
        pooled, ids = self._pool_to_latents(x)
        gk, gv = (t.transpose(1, 2) for t in self.rkv_proj(pooled).view(B, pooled.size(1), 2, Lh, Ldh)
                  .unbind(dim=2))
        if self.latent_query_block_size > 1:
            qsrc, qids = self._pool_query_blocks(x, ids)
        else:
            qsrc, qids = x, ids
        nq = qsrc.size(1)
        rq = self.rq_proj(qsrc).view(B, nq, Lh, Ldh).transpose(1, 2)
        local = self._local_attention(q, k, v)
        # the latent products are tiny (Nc latents per query); they run in fp32 so that no bf16 batched product
        # with a transposed operand is issued on the GPU (see _sdpa)
        with torch.autocast(device_type=x.device.type, enabled=False):
            wide = torch.promote_types(rq.dtype, torch.float32)
            rq32, gk32, gv32 = rq.to(wide), gk.to(wide), gv.to(wide)
            scores = torch.matmul(rq32, gk32.transpose(-2, -1)) / math.sqrt(Ldh)
            causal = torch.arange(pooled.size(1), device=x.device).unsqueeze(0) >= qids.unsqueeze(1)
            scores = scores.masked_fill(causal.unsqueeze(0).unsqueeze(0), float("-inf"))
            valid = (~causal).any(dim=-1).view(1, 1, nq, 1)
            scores = torch.where(valid, scores, torch.zeros_like(scores))
            lat = torch.matmul(torch.softmax(scores, dim=-1) * valid, gv32).to(rq.dtype)
        remote = self.r_out(lat.transpose(1, 2).contiguous().view(B, nq, Lh * Ldh))
        if self.latent_query_block_size > 1:
            qb = min(T, self.latent_query_block_size)
            reps = torch.full((nq,), qb, dtype=torch.long, device=x.device)
            if T % qb:
                reps[-1] = T % qb
            remote = torch.repeat_interleave(remote, reps, dim=1)
        remote = remote.view(B, T, H, Dh).transpose(1, 2)
        s_l, s_r = self.gate_local(local), self.gate_remote(remote)
        m = torch.maximum(s_l, s_r)
        e_l, e_r = torch.exp(s_l - m), torch.exp(s_r - m)
        z = e_l + e_r
        mixed = (e_l / z) * local + (e_r / z) * remote
        return self.out(mixed.transpose(1, 2).contiguous().view(B, T, D))


class TorchRMSNorm(nn.Module):
    """The reference's RMSNorm (reference models.py:40-47, ``F.rms_norm``): the norm of the config-5
    comparison model."""

    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        return F.rms_norm(x, (self.weight.shape[0],), self.weight, self.eps)


def lm_flops(c):
    """Algorithmic FLOPs of one training step of the LM: 3 x forward (sum of 2 M N K over the contractions;
    the attention layers as module_flops, the FFN, the tied head)."""
    lay = layout(CONFIGS["c2"] | {k: c[k] for k in ("B", "T")})
    tokens = c["B"] * c["T"]
    ffn = 2 * 2 * c["d_model"] * c["d_ff"]
    head = 2 * c["d_model"] * c["vocab"]
    return c["n_layers"] * module_flops(lay) + 3 * tokens * (c["n_layers"] * ffn + head)


def bench_lm(args):
    """Config 5: one bf16 AdamW training step of the 0.55b LocalLatentLM (22 layers, the HIP block and the
    HIP RMSNorm in every layer), tokens/s, next to the reference model (PyTorch SDPA + eager latent block,
    torch RMSNorm) with the same weights on the same GPU."""
    from llattn_amd.lm import build_model, make_optimizer, train_step

    c = LM_CONFIG
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(5)
    tokens = torch.randint(0, c["vocab"], (c["B"], c["T"] + 1), device=dev, generator=g)
    inputs, targets = tokens[:, :-1], tokens[:, 1:]
    kw = dict(vocab_size=c["vocab"], max_seq_len=c["T"])

    def run(model, label, fused):
        opt = make_optimizer(model)
        first = float(train_step(model, opt, inputs, targets, fused_loss=fused))
        for _ in range(args.warmup - 1):
            train_step(model, opt, inputs, targets, fused_loss=fused)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            loss = train_step(model, opt, inputs, targets, fused_loss=fused)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1000.0 / args.steps
        log(f"{label}: {ms:.2f} ms per step, first-step loss {first:.5f}, last loss {float(loss):.5f}, "
            f"peak memory {torch.cuda.max_memory_allocated() / 2**30:.1f} GiB")
        return ms, first

    torch.manual_seed(0)
    model = build_model("0.55b", **kw).to(dev)
    init = {k: v.detach().clone() for k, v in model.state_dict().items()}
    ms, first = run(model, "HIP block", True)
    ntok = c["B"] * c["T"]
    flops = lm_flops(c)
    if args.no_sdpa_baseline:
        ms_ref = first_ref = None
    else:
        del model
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        ref = build_model("0.55b", attention_factory=TorchPathAttention, norm_factory=TorchRMSNorm, **kw).to(dev)
        for blk in ref.blocks:  # the reference FeedForward: torch GEMMs and a separate GELU
            blk.ff.fused = False
        ref.load_state_dict(init)
        del init
        ms_ref, first_ref = run(ref, "PyTorch SDPA + eager latent block", False)
    result = {
        "metric": "LocalLatentLM 0.55b bf16 training step tokens/s (forward, backward, AdamW)",
        "value": round(ntok / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (tokens uniform in [0, 32000), seeded; next-token targets; LocalLatentLM init)",
        "config": {"workload": "0.55b LocalLatentLM training step, HIP block in all 22 layers (BASELINE config 5)",
                   "batch": c["B"], "seq_len": c["T"], "vocab": c["vocab"], "layers": c["n_layers"],
                   "d_model": c["d_model"], "d_ff": c["d_ff"], "parallelism": "none (1 GPU)",
                   "precision": "bf16 autocast, fp32 master weights, fused AdamW, grad clip 1.0",
                   "loss": "tied head + cross entropy in chunks of 8192 rows (llattn_xent)"},
        "mfma_frac_step": round(flops / (ms * 1e-3) / MFMA_BF16_PEAK, 4),
        "step_tflop": round(flops / 1e12, 3),
    }
    if ms_ref is not None:
        result["sdpa_baseline"] = {
            "value": round(ntok / (ms_ref * 1e-3), 1), "unit": "tokens/s", "ms_per_step": round(ms_ref, 3),
            "what": "same model and weights with the reference PyTorch attention block (SDPA + eager latent), "
                    "torch RMSNorm and full logits + F.cross_entropy, same GPU, same run"}
        result["sdpa_baseline"]["deviations"] = (
            "SDPA is pinned to its memory-efficient backend for bf16 GPU inputs and the latent attention products "
            "run in fp32: bf16 batched products with a transposed right operand (which SDPA's math path, its "
            "backward and the reference's latent matmuls issue) are documented to fault MI355X boxes under this "
            "software stack, so the reference's own calls are not run as written")
        result["speedup_vs_sdpa"] = round(ms_ref / ms, 3)
        result["first_step_loss"] = {"hip": round(first, 5), "sdpa": round(first_ref, 5)}
    return result


def _board_sample():
    """(socket power W, mean GFX clock MHz) from one ``amd-smi metric --power --clock`` reading, or None."""
    import re
    import subprocess
    try:
        out = subprocess.run(["amd-smi", "metric", "--power", "--clock"], capture_output=True, text=True,
                             timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    p = re.search(r"SOCKET_POWER:\s*([0-9.]+)\s*W", out)
    gfx = out.split("GFX_0:", 1)[1] if "GFX_0:" in out else ""
    # the current clock lines of the GFX_<i> sections (not their MIN_CLK / MAX_CLK lines)
    clk = [float(v) for v in re.findall(r"^\s*CLK:\s*([0-9.]+)\s*MHz", gfx.split("MEM_0:", 1)[0], re.M)]
    if not p or not clk:
        return None
    return float(p.group(1)), sum(clk) / len(clk)


def bench_gemm_products(args):
    """The config-2 step's nine large GEMM products, each timed alone (HIP events, 20 calls after 3 warm-up
    calls) on this library's kernel and on torch's library GEMM (hipBLASLt) with the same bf16 operands;
    then board power and GFX clock sampled by ``amd-smi`` during 4-second loops of the largest product on
    each, and the same for a square 8192 x 8192 x 8192 bf16 product (the board's sustained ceiling on a shape
    with a long k loop, next to the step's K = 1408 products).  Output: one JSON line."""
    import threading

    from llattn_amd import gemm
    from llattn_amd.linear import weight_grad

    dev = torch.device("cuda:0")
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(3)
    M, D, QK, R = 32768, 1408, 4736, 512   # tokens, d_model, 3 D + latent d_model, latent width (r_out)

    def rnd(*s):
        return (torch.randn(*s, device=dev, generator=g) * 0.5).to(bf)

    prods = []
    for name, N, K in (("qkv|rq", QK, D), ("out", D, D), ("r_out", D, R)):
        x, w, b, dy = rnd(M, K), rnd(N, K), torch.randn(N, device=dev, generator=g), rnd(M, N)
        bb = b.to(bf)
        prods += [
            (f"{name} forward x W^T + b", M, N, K, lambda x=x, w=w, b=b: gemm.linear(x, w, b),
             lambda x=x, w=w, bb=bb: F.linear(x, w, bb)),
            (f"{name} input gradient dy W", M, K, N, lambda dy=dy, w=w: gemm.input_grad(dy, w),
             lambda dy=dy, w=w: dy @ w),
            (f"{name} weight gradient dy^T x (+ db)", N, K, M, lambda dy=dy, x=x: weight_grad(dy, x, True),
             lambda dy=dy, x=x: (dy.t() @ x, dy.sum(0))),
        ]

    def timed(fn, n=20):
        for _ in range(3):
            fn()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record()
        for _ in range(n):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) * 1e3 / n

    rows = []
    for name, m, n, k, ours, lib in prods:
        flop = 2.0 * m * n * k
        t_o, t_l = timed(ours), timed(lib)
        rows.append({"product": name, "M": m, "N": n, "K": k, "us": round(t_o, 1), "tflops": round(flop / t_o / 1e6, 1),
                     "library_us": round(t_l, 1), "library_tflops": round(flop / t_l / 1e6, 1)})
        log(f"{name:40s} ours {t_o:7.1f} us {flop / t_o / 1e6:7.1f} TF/s | library {t_l:7.1f} us "
            f"{flop / t_l / 1e6:7.1f} TF/s")

    def sustained(fn, flop, seconds=4.0):
        samples, stop = [], threading.Event()

        def sampler():
            time.sleep(1.0)  # let the clock settle under load
            while not stop.is_set():
                s = _board_sample()
                if s:
                    samples.append(s)
                time.sleep(0.5)

        th = threading.Thread(target=sampler)
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        th.start()
        t0, n = time.perf_counter(), 0
        while time.perf_counter() - t0 < seconds:
            for _ in range(10):
                fn()
            torch.cuda.synchronize()
            n += 10
        dt = time.perf_counter() - t0
        stop.set()
        th.join()
        out = {"tflops": round(flop * n / dt / 1e12, 1), "samples": len(samples)}
        if samples:
            out["power_w"] = round(sum(p for p, _ in samples) / len(samples), 1)
            out["gfx_mhz"] = round(sum(c for _, c in samples) / len(samples), 1)
        return out

    idle = _board_sample()
    _, m, n, k, ours, lib = prods[0]
    power = {"idle": None if idle is None else {"power_w": idle[0], "gfx_mhz": idle[1]},
             "ours qkv|rq forward loop": sustained(ours, 2.0 * m * n * k),
             "library qkv|rq forward loop": sustained(lib, 2.0 * m * n * k)}
    del prods
    S = 8192
    a, b, c = rnd(S, S), rnd(S, S), torch.empty(S, S, device=dev, dtype=bf)
    sq_ours = lambda: gemm.linear(a, b, out=c)  # noqa: E731
    sq_lib = lambda: torch.matmul(a, b.t(), out=c)  # noqa: E731
    ref = torch.matmul(a, b.t()).float()
    sq_err = float((gemm.linear(a, b).float() - ref).abs().max() / ref.abs().max())
    del ref
    flop = 2.0 * S ** 3
    for name, fn in (("ours", sq_ours), ("library", sq_lib)):
        t = timed(fn)
        power[f"{name} 8192^3 loop"] = {"burst_us": round(t, 1), "burst_tflops": round(flop / t / 1e6, 1),
                                       **sustained(fn, flop)}
    power["8192^3 ours vs library max rel"] = sq_err
    log(json.dumps(power))
    tot_o = sum(r["us"] for r in rows)
    tot_l = sum(r["library_us"] for r in rows)
    return {"gemm_products": rows, "total_us": round(tot_o, 1), "library_total_us": round(tot_l, 1),
            "board": power,
            "note": "library = torch F.linear / matmul on the same bf16 operands (hipBLASLt); its weight gradient "
                    "has bf16 output and a separate column sum, ours fp32 output with the bias gradient in the pass"}


def bench_stream_overlap(args):
    """Whether an HBM-bound kernel and a power-bound GEMM gain from running on two streams at once: this
    library's cast (llattn_cast: 128 Mi fp32 -> bf16, 768 MB of traffic) and the config-2 ``out`` weight
    gradient (fp32 dy^T x over 32768 tokens with the bias gradient, split-K), timed back to back on one stream,
    on two streams of the default priority joined by events, and on two streams restricted to disjoint halves
    of the CUs (hipExtStreamCreateWithCUMask).  Wall time per pair over 20 pairs after 3 warm-up pairs."""
    import ctypes

    from llattn_amd.linear import pack_params, weight_grad

    dev = torch.device("cuda:0")
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(11)
    M, D = 32768, 1408
    dy = (torch.randn(M, D, device=dev, generator=g) * 0.5).to(bf)
    x = (torch.randn(M, D, device=dev, generator=g) * 0.5).to(bf)
    big = torch.randn(128 << 20, device=dev, generator=g)

    def gemm_op():
        weight_grad(dy, x, True)

    def hbm_op():
        pack_params([([big], bf)])

    def timed(fn, n=20):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return round((time.perf_counter() - t0) / n * 1e6, 1)

    main = torch.cuda.current_stream()

    def pair(s_hbm, s_gemm):
        def f():
            ev = torch.cuda.Event()
            ev.record(main)
            s_hbm.wait_event(ev)
            s_gemm.wait_event(ev)
            with torch.cuda.stream(s_hbm):
                hbm_op()
            with torch.cuda.stream(s_gemm):
                gemm_op()
            main.wait_stream(s_hbm)
            main.wait_stream(s_gemm)
        return f

    res = {"gemm alone": timed(gemm_op), "hbm alone": timed(hbm_op),
           "one stream (serial)": timed(lambda: (hbm_op(), gemm_op()))}
    s1, s2 = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    res["two streams"] = timed(pair(s1, s2))
    hip = ctypes.CDLL("libamdhip64.so")

    def masked(words):
        s = ctypes.c_void_p()
        arr = (ctypes.c_uint32 * len(words))(*words)
        rc = hip.hipExtStreamCreateWithCUMask(ctypes.byref(s), len(words), arr)
        return torch.cuda.ExternalStream(s.value, device=dev) if rc == 0 else None

    sg, sh = masked([0xFFFFFFFF] * 4 + [0] * 4), masked([0] * 4 + [0xFFFFFFFF] * 4)
    if sg is not None and sh is not None:
        with torch.cuda.stream(sg):
            res["gemm alone, half the CUs"] = timed(gemm_op)
        with torch.cuda.stream(sh):
            res["hbm alone, half the CUs"] = timed(hbm_op)
        res["two streams, disjoint CU halves"] = timed(pair(sh, sg))
    log(json.dumps(res))
    return {"stream_overlap_us": res}


def read_traffic(config: str, kernel: str):
    """HBM bytes per call of the entry point `kernel` at `config`, as measured by the rocprofv3 --pmc
    FETCH_SIZE / WRITE_SIZE runs summarised in profiles/ (scaled by a plain copy), or None."""
    f = REPO / "profiles" / "pmc_traffic.json"
    if not f.exists():
        return None
    try:
        return json.loads(f.read_text()).get(config, {}).get(kernel)
    except (ValueError, OSError, AttributeError):
        return None


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", choices=sorted(CONFIGS) + ["c5"], default="c2",
                    help="c2 (default), c3, c4: one attention layer; c5: a full training step of the 0.55b LM")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-sdpa-baseline", action="store_true", help="c5: time the HIP model only")
    ap.add_argument("--cpu-budget", type=float, default=15.0,
                    help="CPU baseline: three timed passes after the warm-up when it took at most this many seconds")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run 3 plain device copies of MIB MiB each (scale factor for rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE counters) and exit")
    ap.add_argument("--gemm-products", action="store_true",
                    help="only time the config-2 step's GEMM products alone, ours against torch's library GEMM, "
                         "with board power and clock under sustained loops, and exit")
    ap.add_argument("--stream-overlap", action="store_true",
                    help="only time an HBM-bound kernel and a weight-gradient GEMM serial against two streams, "
                         "and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the library drives one GPU per process and has no multi-GPU path)",
              file=sys.stderr)
        sys.exit(2)

    from llattn_amd import ops as llops

    if args.calibrate_copy:
        n = args.calibrate_copy << 20
        src = torch.ones(n // 4, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": n}), flush=True)
        return

    if args.gemm_products:
        print(json.dumps(bench_gemm_products(args)), flush=True)
        return
    if args.stream_overlap:
        print(json.dumps(bench_stream_overlap(args)), flush=True)
        return
    if args.config == "c5":
        print(json.dumps(bench_lm(args)), flush=True)
        return
    cfg = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    lay = layout(cfg)
    m = make_module(cfg, dev)
    g = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn(cfg["B"], cfg["T"], cfg["d_model"], device=dev, generator=g).to(torch.bfloat16)
    x.requires_grad_(True)
    dy = torch.randn(cfg["B"], cfg["T"], cfg["d_model"], device=dev, generator=g).to(torch.bfloat16)

    def step():
        for p in m.parameters():
            p.grad = None
        x.grad = None
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            out = m(x)
        out.backward(dy)

    for _ in range(args.warmup):
        step()
    # Timed region 1: the K steps as a user runs them -> value, ms_per_step.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    # Timed region 2: the same K steps with a HIP event pair on the launch stream around every C-ABI call
    # -> per-entry-point durations for `roofline` / `kernels`.  Each event record costs the GPU about 5 us
    # between kernels, so these steps are not the ones `value` is measured on.
    torch.cuda.synchronize()
    llops.EVENT_LOG = []
    t2 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    events, llops.EVENT_LOG = llops.EVENT_LOG, None
    log(f"step {(t1 - t0) * 1000.0 / args.steps:.3f} ms; with per-call events {(t3 - t2) * 1000.0 / args.steps:.3f} ms")

    ms = (t1 - t0) * 1000.0 / args.steps
    tokens = cfg["B"] * cfg["T"]
    flops = module_flops(lay)
    per_kernel, per_work = {}, {}
    for name, s, e, work in events:
        per_kernel.setdefault(name, []).append(s.elapsed_time(e))
        if work is not None:
            per_work[name] = per_work.get(name, 0) + work
    kb = kernel_bytes(lay, 2)
    kstats = {}
    for name, ts in per_kernel.items():
        avg = sum(ts) / len(ts)
        st = {"avg_ms": round(avg, 4), "launches_per_step": len(ts) / args.steps}
        if name in FLOP_ENTRY_POINTS and name in per_work:  # MFMA-bound: algorithmic FLOPs per launch
            st["alg_tflop"] = round(per_work[name] / len(ts) / 1e12, 6)
            st["achieved_TFLOPs"] = round(per_work[name] / (sum(ts) * 1e-3) / 1e12, 1)
        elif name in kb or name in per_work:  # HBM-bound: algorithmic bytes per launch
            st["alg_bytes"] = kb[name] if name in kb else int(per_work[name] / len(ts))
            st["achieved_GBs"] = round(st["alg_bytes"] / (avg * 1e-3) / 1e9, 1)
        kstats[name] = st
    # the dominant entry point: most time per step
    dom = max(kstats, key=lambda n: kstats[n]["avg_ms"] * kstats[n]["launches_per_step"])
    traffic = read_traffic(args.config, dom)
    if "achieved_TFLOPs" in kstats[dom]:
        ach = kstats[dom]["achieved_TFLOPs"]
        roof = {"kernel": dom, "bound": "mfma", "achieved": ach, "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                "frac": round(ach * 1e12 / MFMA_BF16_PEAK, 4), "traffic": traffic}
    else:
        ach = kstats[dom]["achieved_GBs"]
        roof = {"kernel": dom, "bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic}
    for n, st in sorted(kstats.items(), key=lambda kv: -kv[1]["avg_ms"]):
        log(f"  {n:28s} {st}")
    log(f"step {ms:.3f} ms, HIP entry points {sum(s['avg_ms'] * s['launches_per_step'] for s in kstats.values()):.3f} ms")

    result = {
        "metric": "LL-attn fwd+bwd tokens/s + % MFMA peak, 0.55b layer B16 T2048 bf16",
        "value": round(tokens / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (x, dY ~ N(0,1); LocalLatentLM init, 22-layer preset scaling)",
        "config": {"workload": cfg["workload"], "batch": cfg["B"], "seq_len": cfg["T"], "d_model": cfg["d_model"],
                   "heads": cfg["n_heads"], "head_dim": lay.Dh, "window": cfg["window"], "local_block": lay.block,
                   "latents": lay.n_chunks, "latent_dim": cfg["latent_d_model"], "latent_heads": cfg["latent_heads"],
                   "latent_query_block": lay.q_block, "parallelism": "none (1 GPU)",
                   "precision": "bf16 autocast, fp32 master weights"},
        "mfma_frac_module": round(flops / (ms * 1e-3) / MFMA_BF16_PEAK, 4),
        "module_tflop_per_step": round(flops / 1e12, 4),
        "roofline": roof,
        "kernels": kstats,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, args.cpu_budget)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
