"""GPU parity of the LM-head cross entropy (``llattn_xent``) and the chunked head loss built on it, against the
CPU oracle (oracle/llattn_oracle.py:cross_entropy_rows) and a float32 torch restatement of the reference
training step's head + ``F.cross_entropy`` (reference train.py:354-358, models.py:516-517, 576)."""
import numpy as np
import pytest
import torch

from oracle.llattn_oracle import cross_entropy_rows

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _xent():
    from llattn_amd import xent
    return xent


@pytest.mark.parametrize("V", [1000, 8192, 32000, 65536])
@pytest.mark.parametrize("inplace", [False, True])
def test_xent_rows_match_oracle(V, inplace):
    """Loss, first argmax and the bf16 gradient of every row; ignored rows and an out-of-range target."""
    print(f"xent rows V={V} inplace={inplace}", flush=True)
    xent = _xent()
    g = torch.Generator().manual_seed(V)
    R = 37
    x = (torch.randn(R, V, generator=g) * 3.0).to(torch.bfloat16)
    x[5] = 0.25  # a constant row: every index ties, argmax 0, loss log V
    t = torch.randint(0, V, (R,), generator=g)
    t[3] = -100
    t[7] = V + 5  # outside [0, V): NaN loss
    valid = int(((t != -100)).sum())
    scale = torch.tensor(1.0 / valid, device=DEV)
    xd = x.to(DEV)
    dl = xd if inplace else torch.empty_like(xd)
    loss, pred = xent.xent_rows(xd, t.to(DEV), grad_scale=scale, dlogits=dl)
    torch.cuda.synchronize()
    t_or = t.numpy().copy()
    t_or[7] = -100  # the oracle has no out-of-range rule; that row is checked on its own
    lo, po, go = cross_entropy_rows(x.float().numpy(), t_or)
    loss_c = loss.cpu().numpy()
    assert np.isnan(loss_c[7])
    keep = np.arange(R) != 7
    np.testing.assert_allclose(loss_c[keep], lo[keep], rtol=2e-6, atol=2e-5)
    assert loss_c[3] == 0.0 and loss_c[5] == pytest.approx(np.log(V), rel=1e-6)
    np.testing.assert_array_equal(pred.cpu().numpy(), po)
    grad = dl.float().cpu().numpy()
    want = go * (1.0 / valid)
    want[7] = 0.0
    grad[7] = 0.0  # an out-of-range target's row gradient is unspecified beyond being finite
    np.testing.assert_allclose(grad, want, rtol=8e-3, atol=1e-3 / valid)
    assert (grad[3] == 0).all()


def test_xent_rows_without_gradient_leaves_logits():
    xent = _xent()
    x = torch.randn(9, 4096, device=DEV).to(torch.bfloat16)
    keep = x.clone()
    t = torch.randint(0, 4096, (9,), device=DEV)
    loss, pred = xent.xent_rows(x, t)
    torch.cuda.synchronize()
    assert torch.equal(x, keep)
    lo, po, _ = cross_entropy_rows(x.float().cpu().numpy(), t.cpu().numpy())
    np.testing.assert_allclose(loss.cpu().numpy(), lo, rtol=2e-6, atol=2e-5)
    np.testing.assert_array_equal(pred.cpu().numpy(), po)


def _reference_head_loss(h, w, t):
    """The reference step's head + loss under bf16 autocast, restated in float32: bf16 logits from bf16
    operands, fp32 cross entropy, bf16 logit gradient, GEMMs of the bf16 operands (float32 math)."""
    hb = h.detach().to(torch.bfloat16).float()
    wb = w.detach().to(torch.bfloat16).float()
    logits = (hb @ wb.t()).to(torch.bfloat16).float().requires_grad_(True)
    loss = torch.nn.functional.cross_entropy(logits, t)
    (dlog,) = torch.autograd.grad(loss, logits)
    dlog = dlog.to(torch.bfloat16).float()
    return loss.detach(), logits.detach().argmax(-1), dlog @ wb, dlog.t() @ hb


@pytest.mark.parametrize("N,chunk", [(300, 128), (512, 8192), (2048, 512)])
def test_lm_head_loss_matches_reference_step(N, chunk):
    """Chunked head loss (ragged last chunk, single chunk, several full chunks) against the unchunked
    reference computation: loss, accuracy, hidden-state and weight gradients."""
    print(f"lm_head_loss N={N} chunk={chunk}", flush=True)
    xent = _xent()
    g = torch.Generator().manual_seed(N)
    D, V = 256, 2048
    h = torch.randn(N, D, generator=g).to(DEV)
    w = (torch.randn(V, D, generator=g) * 0.05).to(DEV).requires_grad_(True)
    t = torch.randint(0, V, (N,), generator=g).to(DEV)
    t[::17] = -100
    hq = h.to(torch.bfloat16).requires_grad_(True)
    loss, pred = xent.lm_head_loss(hq, w, t, chunk_rows=chunk)
    loss.backward()
    torch.cuda.synchronize()
    ref_loss, ref_pred, ref_dh, ref_dw = _reference_head_loss(hq, w, t)
    assert float(loss) == pytest.approx(float(ref_loss), rel=1e-4)
    assert (pred == ref_pred).float().mean() > 0.97  # ties and 1-ulp logit differences aside
    for got, want in ((hq.grad.float(), ref_dh), (w.grad, ref_dw)):
        err = (got - want).abs().max() / want.abs().max()
        assert err < 2e-2, float(err)
    assert w.grad.dtype == torch.float32 and hq.grad.dtype == torch.bfloat16


def test_lm_head_loss_upstream_gradient_scales():
    xent = _xent()
    h = torch.randn(256, 128, device=DEV).to(torch.bfloat16).requires_grad_(True)
    w = (torch.randn(512, 128, device=DEV) * 0.05).requires_grad_(True)
    t = torch.randint(0, 512, (256,), device=DEV)
    loss, _ = xent.lm_head_loss(h, w, t)
    (3.0 * loss).backward()
    g3 = w.grad.clone()
    w.grad = None
    loss, _ = xent.lm_head_loss(h, w, t)
    loss.backward()
    torch.testing.assert_close(g3, 3.0 * w.grad, rtol=1e-6, atol=0)


def test_model_loss_matches_logits_path():
    """LocalLatentLM.loss (chunked head) against lm_loss(model(x)) on the same weights, bf16 autocast."""
    from llattn_amd.lm import build_model, lm_loss
    torch.manual_seed(0)
    kw = dict(vocab_size=512, max_seq_len=256, d_model=192, n_heads=2, n_layers=1, d_ff=384, local_window=32,
              local_block_size=64, latent_tokens=8, latent_d_model=64, latent_heads=2)
    model = build_model(**kw).to(DEV)
    inputs = torch.randint(0, 512, (2, 256), device=DEV)
    targets = torch.randint(0, 512, (2, 256), device=DEV)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        l1, m1 = model.loss(inputs, targets, chunk_rows=192)
        l1.backward()
    g1 = {n: p.grad.clone() for n, p in model.named_parameters()}
    model.zero_grad(set_to_none=True)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        l2, m2 = lm_loss(model(inputs), targets)
        l2.backward()
    assert float(l1) == pytest.approx(float(l2), rel=2e-3)
    assert abs(float(m1["eval_acc"]) - float(m2["eval_acc"])) < 0.02
    for n, p in model.named_parameters():
        err = (g1[n] - p.grad).abs().max() / p.grad.abs().max().clamp(min=1e-30)
        assert err < 5e-2, (n, float(err))


def test_xent_smallest_vocab_and_single_row():
    xent = _xent()
    x = torch.tensor([[0.5, -1.0, 2.0, 2.0, 0.0, -3.0, 1.5, 2.0]], device=DEV).to(torch.bfloat16)
    t = torch.tensor([6], device=DEV)
    scale = torch.tensor(1.0, device=DEV)
    d = torch.empty_like(x)
    loss, pred = xent.xent_rows(x, t, grad_scale=scale, dlogits=d)
    lo, po, go = cross_entropy_rows(x.float().cpu().numpy(), t.cpu().numpy())
    assert int(pred[0]) == 2 == int(po[0])  # three-way tie at 2.0: the first index
    assert float(loss[0]) == pytest.approx(float(lo[0]), rel=1e-6)
    np.testing.assert_allclose(d.float().cpu().numpy(), go, rtol=8e-3, atol=1e-3)


def test_lm_head_loss_all_rows_ignored_and_chunk_rounding():
    """Every target ignored: NaN loss (as torch's mean over no rows) and zero gradients; a chunk size that is
    not a multiple of 64 is rounded down to one."""
    xent = _xent()
    h = torch.randn(130, 64, device=DEV).to(torch.bfloat16).requires_grad_(True)
    w = (torch.randn(128, 64, device=DEV) * 0.05).requires_grad_(True)
    t = torch.full((130,), -100, device=DEV)
    loss, _ = xent.lm_head_loss(h, w, t, chunk_rows=100)
    loss.backward()
    assert torch.isnan(loss)
    assert not h.grad.any() and not w.grad.any()
    ref = torch.nn.functional.cross_entropy(torch.randn(130, 128), t.cpu())
    assert torch.isnan(ref)


def test_lm_head_loss_vocab_and_width_not_multiples_of_64():
    """V = 1000 and D = 200 (multiples of 8 only) and a row count that is not a multiple of 64: the GEMMs' K
    tails (D in the logits, V in the hidden-state gradient, the rows in the weight gradient) are masked."""
    xent = _xent()
    g = torch.Generator().manual_seed(8)
    N, D, V = 197, 200, 1000
    hq = torch.randn(N, D, generator=g).to(DEV).to(torch.bfloat16).requires_grad_(True)
    w = (torch.randn(V, D, generator=g) * 0.05).to(DEV).requires_grad_(True)
    t = torch.randint(0, V, (N,), generator=g).to(DEV)
    loss, _ = xent.lm_head_loss(hq, w, t, chunk_rows=128)
    loss.backward()
    ref_loss, _, ref_dh, ref_dw = _reference_head_loss(hq, w, t)
    assert float(loss) == pytest.approx(float(ref_loss), rel=1e-4)
    for got, want in ((hq.grad.float(), ref_dh), (w.grad, ref_dw)):
        assert float((got - want).abs().max() / want.abs().max()) < 2e-2


def test_lm_head_loss_under_no_grad_runs_only_the_forward_products():
    """Under torch.no_grad the head computes no gradients (one logits GEMM per chunk, no input- or weight-
    gradient GEMM, no gradient written by the cross-entropy kernel), though its leaves require grad."""
    from llattn_amd import ops
    xent = _xent()
    h = torch.randn(300, 128, device=DEV).to(torch.bfloat16).requires_grad_(True)
    w = (torch.randn(512, 128, device=DEV) * 0.05).requires_grad_(True)
    t = torch.randint(0, 512, (300,), device=DEV)
    with torch.no_grad():
        ref, _ = xent.lm_head_loss(h, w, t, chunk_rows=128)
    ops.EVENT_LOG = []
    try:
        with torch.no_grad():
            loss, _ = xent.lm_head_loss(h, w, t, chunk_rows=128)
        calls = [(e[0], e[3]) for e in ops.EVENT_LOG]
    finally:
        ops.EVENT_LOG = None
    assert [c[0] for c in calls].count("llattn_gemm") == 3, calls  # 3 chunks of <= 128 rows, forward only
    assert all(wk == n * 512 * 2 for (name, wk), n in zip([c for c in calls if c[0] == "llattn_xent"], (128, 128, 44)))
    assert float(loss) == float(ref) and not loss.requires_grad
