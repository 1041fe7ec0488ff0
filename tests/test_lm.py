"""The language model around the block (config 5): composition, initialisation and training step.

CPU: the LM built by ``llattn_amd.lm`` against the reference LM's golden vectors (``tests/golden/lm_tiny.npz``,
written by importing the reference ``models.py``): state-dict keys, every initialised parameter under the
seed, and -- with the attention evaluated by the oracle -- logits, loss and every gradient.  The config-5
comparison block of ``bench.py`` (the reference PyTorch attention path) against the block golden cases.

GPU: the same LM with the HIP block in every layer against the golden vectors (fp32, 1e-4), and a bf16
training step against the fp32 reference path.
"""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from conftest import E2E_CASES, GOLDEN, load_case

LM_KEYS = ("vocab_size", "max_seq_len", "d_model", "n_heads", "n_layers", "d_ff", "local_window", "local_block_size",
           "latent_tokens", "latent_d_model", "latent_heads", "latent_query_block_size")


def _lm_golden():
    z = np.load(GOLDEN / "lm_tiny.npz", allow_pickle=False)
    meta = json.loads(str(z["meta"]))
    params = {k[2:]: z[k] for k in z.files if k.startswith("p:")}
    grads = {k[2:]: z[k] for k in z.files if k.startswith("g:")}
    return meta, z, params, grads


def _oracle_attention_factory():
    """Attention evaluated by the oracle's torch restatement, with the HIP module's parameters."""
    from llattn_amd import LocalLatentAttentionTriton
    from oracle import torch_ref
    from oracle.llattn_oracle import BlockShape

    class OracleAttention(LocalLatentAttentionTriton):
        def forward(self, x, _positions=None):
            shape = BlockShape(d_model=self.d_model, n_heads=self.n_heads, window=self.window,
                               local_block_size=self.local_block_size, latent_tokens=self.n_latents,
                               latent_d_model=self.latent_dim, latent_heads=self.latent_heads,
                               latent_query_block_size=self.latent_query_block_size)
            return torch_ref.block_forward(dict(self.named_parameters()), x, shape)

    def factory(cfg):
        return OracleAttention(cfg.d_model, cfg.n_heads, cfg.latent_heads, cfg.latent_d_model, cfg.latent_tokens,
                               cfg.local_window, local_block_size=cfg.local_block_size,
                               latent_query_block_size=cfg.latent_query_block_size)
    return factory


def _build(meta, factory=None, norm_factory=None):
    from llattn_amd.lm import build_model
    torch.manual_seed(meta["seed"])
    return build_model(attention_factory=factory, norm_factory=norm_factory, **{k: meta[k] for k in LM_KEYS})


def test_lm_keys_and_init_match_reference_under_seed():
    meta, _, params, _ = _lm_golden()
    m = _build(meta)
    assert list(m.state_dict().keys()) == meta["state_dict_keys"]
    assert [n for n, _ in m.named_parameters()] == meta["param_order"]
    assert m.lm_head.weight is m.embedding.weight
    for n, p in m.named_parameters():
        assert np.array_equal(p.detach().double().numpy(), params[n]), n


def test_lm_forward_backward_matches_reference_with_oracle_attention():
    meta, z, params, grads = _lm_golden()
    import bench
    m = _build(meta, _oracle_attention_factory(), bench.TorchRMSNorm).double()
    m.load_state_dict({k: torch.from_numpy(v) for k, v in params.items()}, strict=False)
    from llattn_amd.lm import lm_loss
    logits = m(torch.from_numpy(z["inputs"]))
    loss, metrics = lm_loss(logits, torch.from_numpy(z["targets"]))
    loss.backward()
    np.testing.assert_allclose(logits.detach().numpy(), z["logits"], rtol=0, atol=1e-10)
    assert abs(float(loss.detach()) - float(z["loss"])) < 1e-12
    assert abs(float(metrics["eval_perplexity"]) - float(np.exp(z["loss"]))) < 1e-9
    for n, p in m.named_parameters():
        np.testing.assert_allclose(p.grad.numpy(), grads[n], rtol=0, atol=1e-10, err_msg=n)


def test_lm_loss_metrics():
    from llattn_amd.lm import lm_loss
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(2, 5, 7, generator=g, dtype=torch.float64)
    targets = torch.randint(0, 7, (2, 5), generator=g)
    loss, mt = lm_loss(logits, targets)
    lp = torch.log_softmax(logits, -1).gather(-1, targets[..., None])[..., 0]
    assert abs(float(loss) + float(lp.mean())) < 1e-12
    assert abs(float(mt["eval_acc"]) - float((logits.argmax(-1) == targets).double().mean())) < 1e-7
    assert abs(float(mt["eval_bpt"]) - float(loss) / np.log(2.0)) < 1e-12


@pytest.mark.parametrize("case", E2E_CASES)
def test_config5_comparison_block_is_the_reference_path(case):
    """bench.py's SDPA + eager latent block (the config-5 baseline) reproduces the reference block."""
    import bench
    from llattn_amd import ModelConfig
    meta, x, dout, params, out_ref, dx_ref, grads_ref = load_case(case)
    cfg = ModelConfig(d_model=meta["d_model"], n_heads=meta["n_heads"], local_window=meta["local_window"],
                      local_block_size=meta["local_block_size"], latent_tokens=meta["latent_tokens"],
                      latent_d_model=meta["latent_d_model"], latent_heads=meta["latent_heads"],
                      latent_query_block_size=meta["latent_query_block_size"])
    blk = bench.TorchPathAttention(cfg).double()
    blk.load_state_dict({k: torch.from_numpy(v) for k, v in params.items()})
    xt = torch.from_numpy(x).requires_grad_(True)
    out = blk(xt)
    out.backward(torch.from_numpy(dout))
    np.testing.assert_allclose(out.detach().numpy(), out_ref, rtol=0, atol=1e-10)
    np.testing.assert_allclose(xt.grad.numpy(), dx_ref, rtol=0, atol=1e-10)
    for n, p in blk.named_parameters():
        np.testing.assert_allclose(p.grad.numpy(), grads_ref[n], rtol=0, atol=1e-10, err_msg=n)


@pytest.mark.gpu
def test_lm_hip_block_matches_reference_fp32():
    from gpu_helpers import assert_fp32_close, require_cuda
    from llattn_amd.lm import lm_loss
    dev = require_cuda()
    meta, z, params, grads = _lm_golden()
    m = _build(meta).to(dev)
    m.load_state_dict({k: torch.tensor(v, dtype=torch.float32) for k, v in params.items()}, strict=False)
    logits = m(torch.from_numpy(z["inputs"]).to(dev))
    loss, _ = lm_loss(logits, torch.from_numpy(z["targets"]).to(dev))
    loss.backward()
    assert_fp32_close(logits.detach().cpu().double().numpy(), z["logits"], "logits")
    assert abs(float(loss.detach()) - float(z["loss"])) < 1e-4
    for n, p in m.named_parameters():
        assert_fp32_close(p.grad.cpu().double().numpy(), grads[n], n)


@pytest.mark.gpu
def test_lm_bf16_training_step_against_fp32_reference_path():
    """A bf16-autocast step of the LM with the HIP block: gradients against the same LM with the reference
    PyTorch block in fp32 (bar raised to twice what that reference path itself reaches under bf16), then a
    few optimiser steps that lower the loss."""
    import bench
    from gpu_helpers import assert_bf16_close, err_stats, require_cuda
    from llattn_amd.lm import build_model, lm_loss, make_optimizer, train_step
    dev = require_cuda()
    kw = dict(vocab_size=256, max_seq_len=256, d_model=192, n_heads=2, n_layers=2, d_ff=384, local_window=32,
              local_block_size=64, latent_tokens=8, latent_d_model=64, latent_heads=2)
    torch.manual_seed(3)
    hip = build_model(**kw).to(dev)
    init = {k: v.detach().clone() for k, v in hip.state_dict().items()}
    g = torch.Generator(device=dev).manual_seed(4)
    ids = torch.randint(0, 256, (2, 257), device=dev, generator=g)
    inputs, targets = ids[:, :-1], ids[:, 1:]

    def grads_of(model, bf16):
        model.zero_grad(set_to_none=True)
        d = next(model.parameters()).device
        with torch.autocast(device_type=d.type, dtype=torch.bfloat16, enabled=bf16):
            loss, _ = lm_loss(model(inputs.to(d)), targets.to(d))
            loss.backward()
        return float(loss), {n: p.grad.detach().double().cpu().numpy() for n, p in model.named_parameters()}

    # the reference path and its bf16 floor run on the CPU
    ref = build_model(attention_factory=bench.TorchPathAttention, norm_factory=bench.TorchRMSNorm, **kw)
    ref.load_state_dict({k: v.cpu() for k, v in init.items()})
    loss_ref, g_ref = grads_of(ref, False)
    _, g_floor = grads_of(ref, True)
    loss_hip, g_hip = grads_of(hip, True)
    assert abs(loss_hip - loss_ref) < 2e-2
    for n in g_ref:
        assert_bf16_close(g_hip[n], g_ref[n], n, floor=err_stats(g_floor[n], g_ref[n]))
    opt = make_optimizer(hip, lr=1e-3)
    losses = [float(train_step(hip, opt, inputs, targets)) for _ in range(4)]
    assert all(np.isfinite(losses)) and losses[-1] < losses[0], losses


@pytest.mark.gpu
def test_c5_full_size_step_against_reference_path_loss():
    """BASELINE config 5 at full size: the 0.55b LocalLatentLM (22 layers, the HIP block in each) at B16 T2048,
    vocab 32000, one bf16 AdamW training step; its loss and every updated parameter are finite.  The forward
    loss of sequence 0 under bf16 autocast lies within 2e-2 of the same weights on the reference path (the
    PyTorch attention block of reference models.py:307-462 and torch RMSNorm), run in fp32 on the CPU."""
    import bench
    from gpu_helpers import require_cuda
    from llattn_amd.lm import build_model, make_optimizer, train_step
    dev = require_cuda()
    V, B, T = 32000, 16, 2048
    print("case: c5 full size build", flush=True)
    torch.manual_seed(0)
    model = build_model("0.55b", vocab_size=V, max_seq_len=T).to(dev)
    init = {k: v.detach().cpu().clone() for k, v in model.state_dict().items()}
    g = torch.Generator(device=dev).manual_seed(5)
    tokens = torch.randint(0, V, (B, T + 1), device=dev, generator=g)
    inputs, targets = tokens[:, :-1], tokens[:, 1:]
    print("case: c5 sequence-0 loss on the GPU", flush=True)
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        loss0, _ = model.loss(inputs[:1], targets[:1])
    loss0 = float(loss0)
    print("case: c5 training step", flush=True)
    opt = make_optimizer(model)
    loss = float(train_step(model, opt, inputs, targets))
    assert np.isfinite(loss) and abs(loss - np.log(V)) < 1.0, loss
    for n, p in model.named_parameters():
        assert torch.isfinite(p).all(), n
        assert p.grad is None or torch.isfinite(p.grad).all(), n
    del model, opt
    torch.cuda.empty_cache()
    print("case: c5 sequence-0 loss on the CPU reference path", flush=True)
    torch.set_num_threads(max(1, torch.get_num_threads()))
    ref = build_model("0.55b", attention_factory=bench.TorchPathAttention, norm_factory=bench.TorchRMSNorm,
                      vocab_size=V, max_seq_len=T)
    ref.load_state_dict(init)
    with torch.no_grad():
        logits = ref(inputs[:1].cpu())
        loss_ref = float(torch.nn.functional.cross_entropy(logits.reshape(-1, V).float(), targets[:1].cpu().reshape(-1)))
    print(f"c5 sequence-0 loss: HIP bf16 {loss0:.5f}, reference fp32 {loss_ref:.5f}", flush=True)
    assert abs(loss0 - loss_ref) < 2e-2


@pytest.mark.gpu
def test_checkpointed_blocks_give_the_same_bits():
    """Activation checkpointing (reference models.py:571-572, the trainer's --checkpoint-blocks, train.py:136): a
    small LocalLatentLM with checkpoint_blocks=True re-runs each HIP block's forward in the backward.  The block's
    forward is pure and deterministic, so one bf16 training step gives the loss and every parameter gradient of
    the same model and tokens without checkpointing, bit for bit (the unfused residual norms that checkpointing
    selects give the same bits as the fused ones)."""
    from gpu_helpers import require_cuda
    from llattn_amd.lm import build_model
    dev = require_cuda()
    kw = dict(vocab_size=384, max_seq_len=512, d_model=256, n_heads=4, n_layers=3, d_ff=512, local_window=64,
              local_block_size=128, latent_tokens=8, latent_d_model=128, latent_heads=2)
    g = torch.Generator(device=dev).manual_seed(11)
    tokens = torch.randint(0, kw["vocab_size"], (2, 385), device=dev, generator=g)
    inputs, targets = tokens[:, :-1], tokens[:, 1:]
    results = []
    for ckpt in (False, True):
        torch.manual_seed(0)
        model = build_model(checkpoint_blocks=ckpt, **kw).to(dev)
        model.train()
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            loss, _ = model.loss(inputs, targets)
            loss.backward()
        results.append((loss.detach().clone(), {n: p.grad.detach().clone() for n, p in model.named_parameters()}))
    (l0, g0), (l1, g1) = results
    assert torch.equal(l0, l1), (float(l0), float(l1))
    assert g0.keys() == g1.keys()
    for n in g0:
        assert torch.equal(g0[n], g1[n]), n


@pytest.mark.gpu
def test_block_under_torch_checkpoint_gives_the_same_bits():
    """One HIP block called through torch.utils.checkpoint(use_reentrant=False) (the call the reference LM makes
    for each block, models.py:571-572) against a plain call: output, input gradient and every parameter gradient
    bit for bit, under bf16 autocast at a macro-block shape and a token-wise one."""
    from torch.utils.checkpoint import checkpoint

    import bench
    from gpu_helpers import require_cuda
    dev = require_cuda()
    for cfg in (dict(B=2, T=1024, d_model=512, n_heads=8, window=64, local_block_size=256, latent_tokens=16,
                     latent_d_model=128, latent_heads=2, qbs=0),
                dict(B=2, T=1024, d_model=512, n_heads=8, window=128, local_block_size=256, latent_tokens=16,
                     latent_d_model=128, latent_heads=2, qbs=64)):
        m = bench.make_module(cfg, dev)
        g = torch.Generator(device=dev).manual_seed(3)
        x0 = torch.randn(cfg["B"], cfg["T"], cfg["d_model"], device=dev, generator=g)
        dy = torch.randn(cfg["B"], cfg["T"], cfg["d_model"], device=dev, generator=g)
        outs = []
        for ckpt in (False, True):
            m.zero_grad(set_to_none=True)
            x = x0.clone().requires_grad_(True)
            with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
                y = checkpoint(m, x, use_reentrant=False) if ckpt else m(x)
            y.backward(dy.to(y.dtype))
            outs.append((y.detach().clone(), x.grad.clone(), {n: p.grad.clone() for n, p in m.named_parameters()}))
        (y0, dx0, g0), (y1, dx1, g1) = outs
        assert torch.equal(y0, y1) and torch.equal(dx0, dx1), cfg
        for n in g0:
            assert torch.equal(g0[n], g1[n]), (n, cfg)


def test_odd_vocabulary_takes_the_full_logits_loss(monkeypatch):
    """A vocabulary the chunked head kernels do not take (50257, GPT-2's: not a multiple of 8) makes
    LocalLatentLM.loss fall back to full logits + lm_loss, as the reference computes it, instead of raising."""
    from llattn_amd import lm, xent
    assert xent.head_supported(32000, 1408) and not xent.head_supported(50257, 1408)
    assert not xent.head_supported(70000, 1408) and not xent.head_supported(32000, 100)
    model = lm.build_model(vocab_size=50257, max_seq_len=16, d_model=64, n_heads=2, n_layers=1, d_ff=128,
                           local_window=8, local_block_size=8, latent_tokens=2, latent_d_model=16, latent_heads=2)
    seen = []
    monkeypatch.setattr(lm.LocalLatentLM, "hidden", lambda self, ids: torch.zeros(*ids.shape, 64))
    monkeypatch.setattr(xent, "lm_head_loss", lambda *a, **k: seen.append("chunked"))
    real = lm.lm_loss
    monkeypatch.setattr(lm, "lm_loss", lambda logits, t: (seen.append("full"), real(logits, t))[1])
    ids = torch.randint(0, 50257, (1, 16))
    loss, _ = model.loss(ids, ids)
    assert seen == ["full"] and abs(float(loss) - float(np.log(50257))) < 1e-3


def _oracle_lm(meta, params):
    import bench
    m = _build(meta, _oracle_attention_factory(), bench.TorchRMSNorm).double()
    m.load_state_dict({k: torch.from_numpy(v) for k, v in params.items()}, strict=False)
    return m.eval()


def test_generate_loop_matches_manual_reforward_on_cpu():
    """LocalLatentLM.generate against a literal replay of reference generate.py:188-190 (context = the last
    max_seq_len tokens, full forward, argmax of the last position) on the oracle LM in float64; the prompt
    of 60 tokens grows past max_seq_len = 64, so the context is cropped in the last steps."""
    meta, z, params, _ = _lm_golden()
    m = _oracle_lm(meta, params)
    prompt = torch.from_numpy(z["inputs"][:1, :60])
    got = m.generate(prompt, max_new_tokens=8)
    ids = prompt
    with torch.no_grad():
        for _ in range(8):
            logits = m(ids[:, -meta["max_seq_len"]:])
            ids = torch.cat([ids, logits[:, -1].argmax(-1, keepdim=True)], dim=1)
    assert got.shape == (1, 68) and torch.equal(got, ids)
    # the tied head on the last position alone equals the last row of the full logits
    with torch.no_grad():
        np.testing.assert_allclose(m.next_token_logits(prompt).numpy(), m(prompt)[:, -1].numpy(), rtol=0, atol=1e-12)


@pytest.mark.gpu
def test_generation_replay_on_hip_lm_matches_reference():
    """Reference generate.py:188-190 (a full re-forward of the context per new token) on the lm_tiny LM with
    the HIP block in fp32: teacher-forced over prefixes of golden sequence 0, every step's last-position logits
    match the oracle LM on the same prefix (1e-4), the full-length step matches the reference's golden logits,
    and greedy decoding from a 58-token prompt (cropped at max_seq_len = 64) picks the oracle's tokens.  The
    forward-only path runs: the local kernel gets no o_local / lse / w to write."""
    from gpu_helpers import assert_fp32_close, require_cuda
    from llattn_amd import ops
    dev = require_cuda()
    meta, z, params, _ = _lm_golden()
    ref = _oracle_lm(meta, params)
    hip = _build(meta).to(dev).eval()
    hip.load_state_dict({k: torch.tensor(v, dtype=torch.float32) for k, v in params.items()}, strict=False)
    seq = torch.from_numpy(z["inputs"][:1])
    seen = []
    real_call = ops._call

    def spy(name, *args, **kw):
        if name == "llattn_local_gate_fwd":
            seen.append(args[8:11])  # o_local, lse, w
        return real_call(name, *args, **kw)
    ops._call = spy
    try:
        for t in range(40, seq.shape[1] + 1, 3):
            ctx = seq[:, :t]
            got = hip.next_token_logits(ctx.to(dev)).double().cpu().numpy()
            with torch.no_grad():
                want = ref.next_token_logits(ctx).numpy()
            assert_fp32_close(got, want, f"prefix {t}")
        got = hip.next_token_logits(seq.to(dev)).double().cpu().numpy()
        assert_fp32_close(got, z["logits"][:1, -1], "full sequence vs golden logits")
        gen = hip.generate(seq[:, :58].to(dev), max_new_tokens=10).cpu()
    finally:
        ops._call = real_call
    assert seen and all(s == (None, None, None) for s in seen)
    assert torch.equal(gen, ref.generate(seq[:, :58], max_new_tokens=10))
