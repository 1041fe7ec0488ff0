"""Write the golden vectors that pin the CPU oracle to the reference.

Run once, in the build container (the only place the reference exists):

    python tests/golden/make_golden.py /root/reference

It imports the reference's ``models.py`` on CPU (read-only, no bytecode
written) and records input/output vectors of the functions no closed form
pins on its own:

* ``keyset.npz``   -- the local key set of ``_local_attention`` +
  ``_block_local_mask`` (models.py:232-305), read out through SDPA by
  feeding q = 0 (uniform scores) and one-hot values, for several
  (T, window, local_block_size);
* ``pool.npz``     -- ``_pool_to_latents`` (models.py:159-214) and
  ``_pool_query_blocks`` (models.py:216-230) outputs and index maps;
* ``case_<name>.npz`` -- end-to-end ``LocalLatentAttention.forward``
  (models.py:307-462) output and autograd gradients of x and every
  parameter for ``sum(out * dout)``, float64, inputs stored in full;
* ``case_c1.npz``  -- BASELINE config 1 in float32 (B2 T512 D256 4x64, W128,
  8 latents, latent_dim 32, token-wise).  Its inputs are NOT stored: they
  are regenerated from ``torch.manual_seed(0)`` in this order -- the block's
  parameters in ``LocalLatentAttention.__init__`` order with torch default
  ``nn.Linear`` init, then ``x = randn(2,512,256)``, then
  ``dout = randn(2,512,256)`` -- and the file keeps per-tensor sums so a
  regeneration can be verified.

* ``lm_tiny.npz``   -- a 2-layer ``LocalLatentLM`` (models.py:490-580) built
  under ``torch.manual_seed(21)`` in float64: every initialised parameter,
  input ids and next-token targets, logits, the mean cross entropy and the
  autograd gradient of every parameter (the tied head shares the token
  embedding's).  Pins the LM composition, the module / RNG order of its
  initialisation and the state-dict keys.

Only data is written here; nothing from the reference's source is kept.
``python tests/golden/make_golden.py /root/reference lm`` rewrites only the
LM fixture.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

OUT_DIR = Path(__file__).resolve().parent

PARAM_ORDER = (
    "qkv_proj.weight", "qkv_proj.bias", "rq_proj.weight", "rq_proj.bias",
    "rkv_proj.weight", "rkv_proj.bias", "r_out.weight", "r_out.bias",
    "out.weight", "out.bias", "gate_local.weight", "gate_remote.weight",
)

# (name, dict(ModelConfig fields), B, T, seed)
E2E_CASES = [
    ("tiny_tok", dict(d_model=64, n_heads=2, local_window=16, local_block_size=32, latent_tokens=6,
                      latent_d_model=16, latent_heads=2, latent_query_block_size=0), 2, 97, 11),
    ("tiny_macro", dict(d_model=64, n_heads=2, local_window=16, local_block_size=32, latent_tokens=6,
                        latent_d_model=16, latent_heads=2, latent_query_block_size=24), 2, 97, 12),
    ("w1_chunk1", dict(d_model=32, n_heads=2, local_window=1, local_block_size=8, latent_tokens=64,
                       latent_d_model=16, latent_heads=1, latent_query_block_size=0), 1, 40, 13),
    ("dh88_single_block", dict(d_model=88, n_heads=1, local_window=64, local_block_size=256, latent_tokens=50,
                               latent_d_model=32, latent_heads=4, latent_query_block_size=0), 1, 50, 14),
    ("qbs1_is_tokenwise", dict(d_model=64, n_heads=4, local_window=8, local_block_size=4, latent_tokens=5,
                               latent_d_model=32, latent_heads=2, latent_query_block_size=1), 1, 33, 15),
    ("macro_ragged", dict(d_model=96, n_heads=3, local_window=20, local_block_size=16, latent_tokens=7,
                          latent_d_model=24, latent_heads=3, latent_query_block_size=10), 2, 61, 16),
]

KEYSET_CASES = [(97, 16, 32), (40, 1, 8), (50, 64, 256), (130, 7, 10), (64, 20, 16), (33, 8, 4), (1, 4, 256)]
POOL_CASES = [(97, 6, 0), (97, 6, 24), (40, 64, 0), (16, 16, 0), (130, 128, 0), (61, 7, 10), (5, 3, 2),
              (1, 16, 0), (2048, 16, 0), (100, 16, 64)]


def _import_reference(ref_root: Path):
    sys.dont_write_bytecode = True
    sys.path.insert(0, str(ref_root))
    import models  # noqa: E402  (the reference's models.py)
    return models


def _keyset(models, T: int, W: int, lbs: int) -> np.ndarray:
    cfg = models.ModelConfig(d_model=T, n_heads=1, local_window=W, local_block_size=lbs)
    blk = models.LocalLatentAttention(cfg).double()
    q = torch.zeros(1, 1, T, T, dtype=torch.float64)
    k = torch.zeros(1, 1, T, T, dtype=torch.float64)
    v = torch.eye(T, dtype=torch.float64).view(1, 1, T, T)
    with torch.no_grad():
        o = blk._local_attention(q, k, v)[0, 0]
    allowed = o > 0
    # every allowed key got equal weight 1/|K(i)|; check it to be sure the read-out is exact
    cnt = allowed.sum(dim=1).clamp(min=1).to(torch.float64)
    assert torch.allclose(o, allowed.to(torch.float64) / cnt[:, None]), "key-set read-out not uniform"
    return allowed.numpy()


def write_keysets(models):
    out = {}
    for T, W, lbs in KEYSET_CASES:
        out[f"T{T}_W{W}_bs{lbs}"] = np.packbits(_keyset(models, T, W, lbs), axis=1)
    np.savez_compressed(OUT_DIR / "keyset.npz", **out)


def write_pools(models):
    out = {}
    rng = np.random.default_rng(5)
    for T, ntok, qbs in POOL_CASES:
        D = 4
        cfg = models.ModelConfig(d_model=D, n_heads=1, latent_tokens=ntok, latent_query_block_size=qbs)
        blk = models.LocalLatentAttention(cfg).double()
        x = torch.from_numpy(rng.standard_normal((2, T, D)))
        with torch.no_grad():
            pooled, ids = blk._pool_to_latents(x)
            key = f"T{T}_n{ntok}_q{qbs}"
            out[key + "_x"] = x.numpy()
            out[key + "_pooled"] = pooled.numpy()
            out[key + "_ids"] = ids.numpy()
            if qbs > 1:
                qp, qids = blk._pool_query_blocks(x, ids)
                out[key + "_qpooled"] = qp.numpy()
                out[key + "_qids"] = qids.numpy()
    np.savez_compressed(OUT_DIR / "pool.npz", **out)


def _run_block(blk, x, dout):
    x = x.clone().requires_grad_(True)
    out = blk(x)
    out.backward(dout)
    grads = {n: p.grad.detach().clone() for n, p in blk.named_parameters()}
    return out.detach(), x.grad.detach(), grads


def write_e2e(models):
    for name, cfg_kw, B, T, seed in E2E_CASES:
        torch.manual_seed(seed)
        cfg = models.ModelConfig(**cfg_kw)
        blk = models.LocalLatentAttention(cfg).double()
        # non-trivial gate/bias values so every term is exercised
        with torch.no_grad():
            for n, p in blk.named_parameters():
                if n.endswith("bias") or n.startswith("gate"):
                    p.normal_(0.0, 0.5)
        x = torch.randn(B, T, cfg.d_model, dtype=torch.float64)
        dout = torch.randn(B, T, cfg.d_model, dtype=torch.float64)
        out, dx, grads = _run_block(blk, x, dout)
        arrays = {"x": x.numpy(), "dout": dout.numpy(), "out": out.numpy(), "dx": dx.numpy()}
        for n, p in blk.named_parameters():
            arrays["p:" + n] = p.detach().numpy()
            arrays["g:" + n] = grads[n].numpy()
        meta = dict(cfg_kw, B=B, T=T, seed=seed, dtype="float64", torch=torch.__version__)
        np.savez_compressed(OUT_DIR / f"case_{name}.npz", meta=json.dumps(meta), **arrays)


def write_c1(models):
    cfg_kw = dict(d_model=256, n_heads=4, local_window=128, local_block_size=256, latent_tokens=8,
                  latent_d_model=32, latent_heads=2, latent_query_block_size=0)
    torch.manual_seed(0)
    blk = models.LocalLatentAttention(models.ModelConfig(**cfg_kw))
    x = torch.randn(2, 512, 256)
    dout = torch.randn(2, 512, 256)
    out, dx, grads = _run_block(blk, x, dout)
    sums = {"x": float(x.double().sum()), "dout": float(dout.double().sum())}
    for n, p in blk.named_parameters():
        sums["p:" + n] = float(p.detach().double().sum())
    arrays = {"out": out.numpy(), "dx": dx.numpy()}
    for n in PARAM_ORDER:
        arrays["g:" + n] = grads[n].numpy()
    meta = dict(cfg_kw, B=2, T=512, seed=0, dtype="float32", torch=torch.__version__, input_sums=sums,
                param_order=list(n for n, _ in blk.named_parameters()))
    np.savez_compressed(OUT_DIR / "case_c1.npz", meta=json.dumps(meta), **arrays)


LM_CASE = dict(vocab_size=96, max_seq_len=64, d_model=64, n_heads=2, n_layers=2, d_ff=128, local_window=16,
               local_block_size=32, latent_tokens=6, latent_d_model=16, latent_heads=2, latent_query_block_size=0)


def write_lm(models):
    torch.manual_seed(21)
    model = models.build_model(**LM_CASE).double()
    g = torch.Generator().manual_seed(22)
    ids = torch.randint(0, LM_CASE["vocab_size"], (2, 62), generator=g)
    inputs, targets = ids[:, :-1], ids[:, 1:]
    logits = model(inputs)
    loss = torch.nn.functional.cross_entropy(logits.reshape(-1, logits.size(-1)), targets.reshape(-1))
    loss.backward()
    arrays = {"inputs": inputs.numpy(), "targets": targets.numpy(), "logits": logits.detach().numpy(),
              "loss": loss.detach().numpy()}
    for n, p in model.named_parameters():
        arrays["p:" + n] = p.detach().numpy()
        arrays["g:" + n] = p.grad.numpy()
    meta = dict(LM_CASE, seed=21, ids_seed=22, dtype="float64", torch=torch.__version__,
                state_dict_keys=list(model.state_dict().keys()),
                param_order=[n for n, _ in model.named_parameters()])
    np.savez_compressed(OUT_DIR / "lm_tiny.npz", meta=json.dumps(meta), **arrays)


def main(argv):
    ref_root = Path(argv[1] if len(argv) > 1 else "/root/reference")
    torch.set_num_threads(8)
    models = _import_reference(ref_root)
    if len(argv) > 2 and argv[2] == "lm":
        write_lm(models)
        print("lm_tiny.npz", (OUT_DIR / "lm_tiny.npz").stat().st_size)
        return
    write_keysets(models)
    write_pools(models)
    write_e2e(models)
    write_c1(models)
    write_lm(models)
    for f in sorted(OUT_DIR.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main(sys.argv)
