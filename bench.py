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
inside the timed region),
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
    import torch
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


def cpu_baseline(cfg, budget_s: float):
    """The reference PyTorch path (fp32 torch restatement, autograd backward) on the host cores, on one
    sequence of the workload, repeated until ``budget_s`` of CPU time."""
    import torch
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
    x = torch.randn(1, cfg["T"], D, generator=g)
    dout = torch.randn(1, cfg["T"], D, generator=g)
    torch_ref.block_forward_backward(params, x, dout, shape)  # warm-up
    n, t0 = 0, time.perf_counter()
    while True:
        torch_ref.block_forward_backward(params, x, dout, shape)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 200:
            break
    return {"value": round(n * cfg["T"] / el, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{n} fwd+bwd passes of one {cfg['T']}-token sequence (batch row of the workload), fp32, "
                      f"torch CPU restatement of the reference PyTorch path, {el:.1f} s"}


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
    ap.add_argument("--config", choices=sorted(CONFIGS), default="c2")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline work")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run 3 plain device copies of MIB MiB each (scale factor for rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(one process drives one MI355X here; the sharding design is described in DESIGN.md)",
              file=sys.stderr)
        sys.exit(2)

    import torch
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
    torch.cuda.synchronize()
    llops.EVENT_LOG = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    events, llops.EVENT_LOG = llops.EVENT_LOG, None

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
