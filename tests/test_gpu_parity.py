"""GPU parity: the HIP path (through the C ABI) against the reference's golden
vectors and the CPU oracle.

Tolerances (``tests/gpu_helpers.py``): fp32 kernels within 1e-4 max-abs;
bf16 kernels within 2e-2 max-abs and 1e-2 mean-relative of the fp32 /
float64 reference.  Max-abs is taken after dividing by max(1, max|ref|), so it
is absolute for O(1) tensors and relative for large-magnitude weight
gradients (sums over up to 32k tokens).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import E2E_CASES, load_case, shape_from_meta
from gpu_helpers import (assert_bf16_close, assert_fp32_close, assert_within_floor, bf16_floor, build_module, err_stats,
                         reference_bf16_errors, require_cuda,
                         run_module)
from oracle import llattn_oracle as orc

pytestmark = pytest.mark.gpu


def _print_case(*args):
    from gpu_helpers import set_case
    set_case(" ".join(str(a) for a in args))
    print("case:", *args, flush=True)


# ---------------------------------------------------------------- module vs reference golden vectors

@pytest.mark.parametrize("name", E2E_CASES)
def test_module_fp32_matches_reference_golden(name, monkeypatch):
    """The golden cases in fp32, every projection product on llattn_gemm_f32: torch's GEMM entry points raise
    while the block runs, and the event log counts three products per projection (qkv|rq, rkv, r_out, out,
    plus rq_proj in macro-block mode)."""
    from llattn_amd import ops
    dev = require_cuda()
    _print_case("golden fp32", name)
    meta, x, dout, params, out_ref, dx_ref, grads_ref = load_case(name)
    shape = shape_from_meta(meta)
    m = build_module(shape, params, dev)
    ops.EVENT_LOG = []
    try:
        with monkeypatch.context() as mp:
            for mod, attr in ((torch.nn.functional, "linear"), (torch, "mm"), (torch, "matmul"), (torch, "addmm")):
                mp.setattr(mod, attr, _library_gemm)
            out, dx, grads = run_module(m, torch.tensor(x, dtype=torch.float32, device=dev),
                                        torch.tensor(dout, dtype=torch.float32, device=dev))
        calls = [e[0] for e in ops.EVENT_LOG]
    finally:
        ops.EVENT_LOG = None
    macro = meta["latent_query_block_size"] > 1
    assert calls.count("llattn_gemm_f32") == (15 if macro else 12), calls
    assert_fp32_close(out, out_ref, "out")
    assert_fp32_close(dx, dx_ref, "dx")
    for n in grads_ref:
        assert_fp32_close(grads[n], grads_ref[n], n)


def _library_gemm(*args, **kwargs):
    raise AssertionError("a library GEMM ran inside the block")


@pytest.mark.parametrize("name", E2E_CASES)
def test_module_bf16_autocast_matches_reference_golden(name, monkeypatch):
    """The golden cases under bf16 autocast, with every projection product on llattn_gemm: torch's GEMM entry
    points raise while the block runs, and the event log counts three products (forward, input gradient,
    weight gradient) per projection: qkv|rq, rkv, r_out and out, plus rq_proj in macro-block mode."""
    from llattn_amd import ops
    dev = require_cuda()
    _print_case("golden bf16", name)
    meta, x, dout, params, out_ref, dx_ref, grads_ref = load_case(name)
    shape = shape_from_meta(meta)
    m = build_module(shape, params, dev)
    xb = torch.tensor(x, dtype=torch.bfloat16, device=dev)
    ops.EVENT_LOG = []
    try:
        with monkeypatch.context() as mp:
            for mod, attr in ((torch.nn.functional, "linear"), (torch, "mm"), (torch, "matmul"), (torch, "addmm")):
                mp.setattr(mod, attr, _library_gemm)
            out, dx, grads = run_module(m, xb, torch.tensor(dout, dtype=torch.float32, device=dev),
                                        autocast_bf16=True)
        calls = [e[0] for e in ops.EVENT_LOG]
    finally:
        ops.EVENT_LOG = None
    macro = meta["latent_query_block_size"] > 1
    assert calls.count("llattn_gemm") == (15 if macro else 12), calls
    floor = bf16_floor(params, xb.float().cpu().numpy(), dout, shape, grads_ref)
    for n in grads_ref:
        print(f"  {n}: got {err_stats(grads[n], grads_ref[n])} floor {floor[n]}")
    assert_bf16_close(out, out_ref, "out")
    assert_bf16_close(dx, dx_ref, "dx")
    for n in grads_ref:
        assert_bf16_close(grads[n], grads_ref[n], n, floor=floor[n])


def test_config1_fp32_matches_reference_golden(c1_golden):
    dev = require_cuda()
    _print_case("config 1 fp32")
    meta, params, x, dout, out_ref, dx_ref, grads_ref = c1_golden
    shape = orc.BlockShape(d_model=256, n_heads=4, window=128, local_block_size=256, latent_tokens=8,
                           latent_d_model=32, latent_heads=2)
    m = build_module(shape, {k: v.numpy() for k, v in params.items()}, dev)
    out, dx, grads = run_module(m, x.to(dev), dout.to(dev))
    assert_fp32_close(out, out_ref, "out")
    assert_fp32_close(dx, dx_ref, "dx")
    for n in grads_ref:
        assert_fp32_close(grads[n], grads_ref[n], n)


# ---------------------------------------------------------------- op surface vs oracle pieces

def _op_case(B, T, H, Dh, Lh, Ldh, W, lbs, chunk, qbs, seed, dtype, per_head_gate=False):
    """Random inputs of LLAttnFunction and the float64 oracle's outputs and gradients."""
    from llattn_amd import LLAttnFunction
    dev = require_cuda()
    rng = np.random.default_rng(seed)
    Nc = -(-T // chunk)
    qb = min(T, qbs) if qbs > 1 else 1
    nq = -(-T // qb)
    D, Ld = H * Dh, Lh * Ldh
    arr = dict(Q=rng.standard_normal((B, H, T, Dh)), K=rng.standard_normal((B, H, T, Dh)),
               V=rng.standard_normal((B, H, T, Dh)), GQ=rng.standard_normal((B, Lh, nq, Ldh)),
               GK=rng.standard_normal((B, Lh, Nc, Ldh)), GV=rng.standard_normal((B, Lh, Nc, Ldh)),
               gl=rng.standard_normal((H if per_head_gate else 1, Dh)) * 0.5,
               gr=rng.standard_normal((H if per_head_gate else 1, Dh)) * 0.5,
               rw=rng.standard_normal((D, Ld)) / np.sqrt(Ld), rb=rng.standard_normal(D) * 0.3)
    dOut = rng.standard_normal((B, H, T, Dh))
    # round inputs to the kernel dtype so the oracle sees identical values
    tens = {k: torch.tensor(v, dtype=dtype, device=dev) for k, v in arr.items()}
    for k in ("gl", "gr", "rw", "rb"):
        tens[k] = torch.tensor(arr[k], dtype=torch.float32, device=dev)
    arr = {k: t.double().cpu().numpy() for k, t in tens.items()}
    for t in tens.values():
        t.requires_grad_(True)
    out = LLAttnFunction.apply(tens["Q"], tens["K"], tens["V"], tens["GQ"], tens["GK"], tens["GV"], tens["gl"],
                               tens["gr"], tens["rw"], W, chunk, tens["rb"], lbs, qbs)
    dOut_t = torch.tensor(dOut, dtype=dtype, device=dev)
    dOut = dOut_t.double().cpu().numpy()
    out.backward(dOut_t)
    got = {"out": out.detach().double().cpu().numpy()}
    got.update({k: t.grad.double().cpu().numpy() for k, t in tens.items()})

    # oracle
    shape = orc.BlockShape(d_model=D, n_heads=H, window=W, local_block_size=lbs, latent_tokens=Nc,
                           latent_d_model=Ld, latent_heads=Lh, latent_query_block_size=qbs)
    lay = orc.seq_layout(shape, T)
    assert lay.chunk == chunk and lay.n_chunks == Nc
    O, LSE = orc.local_attention(arr["Q"], arr["K"], arr["V"], lay)
    Lat, P = orc.latent_attention(arr["GQ"], arr["GK"], arr["GV"], lay.q_chunk_ids)
    L_flat = Lat.transpose(0, 2, 1, 3).reshape(B, nq, Ld)
    R_q = L_flat @ arr["rw"].T + arr["rb"]
    tok_q = np.arange(T) // lay.qb
    R_tok = R_q[:, tok_q].reshape(B, T, H, Dh).transpose(0, 2, 1, 3)
    gl = arr["gl"] if per_head_gate else np.broadcast_to(arr["gl"], (H, Dh))
    gr = arr["gr"] if per_head_gate else np.broadcast_to(arr["gr"], (H, Dh))
    s_l = np.einsum("bhtd,hd->bht", O, gl)
    s_r = np.einsum("bhtd,hd->bht", R_tok, gr)
    w = 1.0 / (1.0 + np.exp(-(s_l - s_r)))
    Y = w[..., None] * O + (1 - w[..., None]) * R_tok
    delta = w * (1 - w) * np.einsum("bhtd,bhtd->bht", dOut, O - R_tok)
    dO = w[..., None] * dOut + delta[..., None] * gl[None, :, None, :]
    dR_tok = (1 - w)[..., None] * dOut - delta[..., None] * gr[None, :, None, :]
    dgl = np.einsum("bht,bhtd->hd", delta, O)
    dgr = -np.einsum("bht,bhtd->hd", delta, R_tok)
    if not per_head_gate:
        dgl, dgr = dgl.sum(0, keepdims=True), dgr.sum(0, keepdims=True)
    dR_flat = dR_tok.transpose(0, 2, 1, 3).reshape(B, T, D)
    dR_q = np.zeros((B, nq, D))
    np.add.at(dR_q, (slice(None), tok_q), dR_flat)
    dL = (dR_q @ arr["rw"]).reshape(B, nq, Lh, Ldh).transpose(0, 2, 1, 3)
    drq, dgk, dgv = orc.latent_attention_backward(arr["GQ"], arr["GK"], arr["GV"], Lat, P, dL)
    dq, dk, dv = orc.local_attention_backward(arr["Q"], arr["K"], arr["V"], O, LSE, dO, lay)
    ref = dict(out=Y, Q=dq, K=dk, V=dv, GQ=drq, GK=dgk, GV=dgv, gl=dgl, gr=dgr,
               rw=np.einsum("bsk,bsl->kl", dR_q, L_flat), rb=dR_q.sum((0, 1)))
    if dtype == torch.bfloat16:
        # Precision floor of the gate gradients: the same sums over O and R rounded to bf16, the storage
        # type the bf16 path (like the reference under autocast) keeps them in.  These are sums over all
        # tokens of delta * O with cancellation, so their relative error is set by that rounding.
        def bf(a):
            return torch.tensor(a).to(torch.bfloat16).double().numpy()
        Ob, Rb = bf(O), bf(R_tok)
        wb = 1.0 / (1.0 + np.exp(-(np.einsum("bhtd,hd->bht", Ob, gl) - np.einsum("bhtd,hd->bht", Rb, gr))))
        db = wb * (1 - wb) * np.einsum("bhtd,bhtd->bht", dOut, Ob - Rb)
        fl, fr = np.einsum("bht,bhtd->hd", db, Ob), -np.einsum("bht,bhtd->hd", db, Rb)
        if not per_head_gate:
            fl, fr = fl.sum(0, keepdims=True), fr.sum(0, keepdims=True)
        ref["_floor"] = {"gl": err_stats(fl, dgl), "gr": err_stats(fr, dgr)}
    return got, ref


OP_CASES = [
    # B, T, H, Dh, Lh, Ldh, W, lbs, chunk, qbs
    (2, 97, 2, 32, 2, 8, 16, 32, 17, 0),
    (1, 200, 3, 88, 2, 16, 64, 256, 13, 0),
    (2, 130, 2, 64, 1, 32, 7, 10, 3, 0),
    (1, 160, 2, 128, 4, 16, 100, 64, 40, 0),
    (1, 75, 2, 64, 2, 64, 1, 8, 5, 0),
    (2, 150, 2, 32, 2, 32, 40, 64, 10, 16),
    (1, 61, 4, 16, 2, 8, 20, 16, 9, 10),
    (1, 300, 1, 96, 2, 32, 300, 300, 1, 0),
    (1, 140, 2, 32, 1, 128, 20, 32, 2, 0),      # latent head dim 128, 70 latents (two latent tiles)
    (1, 1100, 1, 32, 1, 16, 16, 64, 8, 0),      # 3 query segments x 9 latent tiles in the latent backward
    (2, 700, 2, 64, 2, 32, 48, 128, 7, 9),      # macro-block queries over several query tiles
    # fused bf16 backward (W <= 64) with local blocks >= 64 that are not multiples of 64: 64-row query
    # tiles that straddle a block boundary (the qr0 + row >= block branch of its key bounds)
    (1, 400, 2, 64, 2, 32, 48, 100, 10, 0),
    (2, 333, 2, 88, 2, 16, 64, 96, 7, 0),
    # wide-window bf16 backward (W > 64): several local blocks per sequence (the first
    # query of each block loses its farthest key), ragged T, macro-block queries, a last 128-key group
    # holding one key, windows that are not multiples of 32, a long window over several key groups
    (2, 333, 2, 64, 2, 32, 100, 64, 11, 0),
    (1, 700, 2, 32, 2, 16, 300, 128, 9, 0),
    (2, 520, 2, 64, 2, 32, 130, 256, 13, 16),
    (1, 129, 1, 64, 1, 16, 65, 65, 5, 0),
    (1, 1000, 1, 64, 2, 32, 512, 256, 20, 0),
    (2, 400, 2, 88, 2, 16, 130, 256, 10, 0),   # 0.55b head dim (padded to 96) with a window above 64
]


# bf16 head dims above 128 (padded to 256) on the generic tile kernels: local forward and two-pass backward,
# latent forward and backward; a window below and above 64, macro-block queries, a ragged head dim
WIDE_HEAD_CASES = [
    (2, 150, 2, 256, 2, 256, 40, 64, 10, 0),
    (1, 200, 2, 160, 1, 192, 100, 64, 13, 16),
    (1, 97, 1, 136, 2, 24, 300, 300, 7, 0),
]


@pytest.mark.parametrize("case", WIDE_HEAD_CASES)
def test_op_bf16_wide_head_dims_match_oracle(case):
    _print_case("op bf16 wide head", case)
    got, ref = _op_case(*case, seed=hash(case) % 1000 + 2, dtype=torch.bfloat16)
    floor = ref.pop("_floor")
    for k in ref:
        assert_bf16_close(got[k], ref[k], k, floor=floor.get(k))


def test_module_bf16_head_dim_256_matches_fp32_reference():
    """A block with 256-dim heads (d_model 512, 2 heads; 2 latent heads of 128) under bf16 autocast against the
    fp32 reference: the projections, head layouts and the 256-dim tile kernels together
    (reference models.py:64-74 accepts any divisible head split)."""
    from oracle import torch_ref
    dev = require_cuda()
    _print_case("module bf16 head dim 256")
    shape = orc.BlockShape(d_model=512, n_heads=2, window=96, local_block_size=128, latent_tokens=16,
                           latent_d_model=256, latent_heads=2)
    torch.manual_seed(11)
    m = build_module(shape, None, dev)
    with torch.no_grad():
        for p in m.parameters():
            p.normal_(0.0, 0.03)
    x = torch.randn(2, 256, 512, device=dev).to(torch.bfloat16)
    dout = torch.randn(2, 256, 512, device=dev)
    out, dx, grads = run_module(m, x, dout, autocast_bf16=True)
    params = {n: p.detach().float().cpu() for n, p in m.named_parameters()}
    o_ref, dx_ref, g_ref = torch_ref.block_forward_backward(params, x.float().cpu(), dout.float().cpu(), shape)
    assert_bf16_close(out, o_ref.numpy(), "out")
    assert_bf16_close(dx, dx_ref.numpy(), "dx")
    for n in g_ref:
        assert_bf16_close(grads[n], g_ref[n].numpy(), n)


@pytest.mark.parametrize("case", OP_CASES)
def test_op_fp32_matches_oracle(case):
    _print_case("op fp32", case)
    got, ref = _op_case(*case, seed=hash(case) % 1000, dtype=torch.float32)
    for k in ref:
        assert_fp32_close(got[k], ref[k], k)


@pytest.mark.parametrize("case", OP_CASES)
def test_op_bf16_matches_oracle(case):
    _print_case("op bf16", case)
    got, ref = _op_case(*case, seed=hash(case) % 1000 + 1, dtype=torch.bfloat16)
    floor = ref.pop("_floor")
    for k in ref:
        assert_bf16_close(got[k], ref[k], k, floor=floor.get(k))


def test_op_per_head_gate():
    _print_case("op per-head gate")
    got, ref = _op_case(2, 90, 3, 32, 3, 8, 12, 24, 10, 0, seed=5, dtype=torch.float32, per_head_gate=True)
    for k in ref:
        assert_fp32_close(got[k], ref[k], k)


@pytest.mark.parametrize("case", [(2, 300, 3, 64, 2, 16, 96, 128, 10, 0), (1, 260, 2, 32, 2, 8, 70, 70, 13, 20)])
def test_op_per_head_gate_bf16(case):
    """Per-head gate vectors on the bf16 kernels: the 32x32 forward and, with windows above 64, the wide-window
    backward, whose gate partial sums are kept per head (fused W <= 64 path: the C2 cases)."""
    _print_case("op per-head gate bf16", case)
    got, ref = _op_case(*case, seed=7, dtype=torch.bfloat16, per_head_gate=True)
    floor = ref.pop("_floor")
    for k in ref:
        assert_bf16_close(got[k], ref[k], k, floor=floor.get(k))


# ---------------------------------------------------------------- pooling op vs reference golden

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_pool_matches_reference_golden(dtype):
    from conftest import GOLDEN
    from llattn_amd import DIV_COUNT, DIV_SEG, pool
    dev = require_cuda()
    z = np.load(GOLDEN / "pool.npz")
    keys = sorted({k.rsplit("_", 1)[0] for k in z.files})
    for key in keys:
        _print_case("pool", key, dtype)
        T, ntok, qbs = (int(t[1:]) for t in key.split("_"))
        shape = orc.BlockShape(d_model=8, n_heads=1, window=4, latent_tokens=ntok, latent_query_block_size=qbs)
        lay = orc.seq_layout(shape, T)
        x = torch.tensor(np.repeat(z[key + "_x"], 2, axis=2), dtype=dtype, device=dev)  # D=8: one 16-byte bf16 vector
        xr = x.double().cpu().numpy()
        ref = orc.pool_segments(xr, lay.chunk, lay.n_chunks, "count")
        got = pool(x, lay.chunk, lay.n_chunks, DIV_COUNT).double().cpu().numpy()
        (assert_fp32_close if dtype == torch.float32 else assert_bf16_close)(got, ref, key)
        if qbs > 1:
            ref = orc.pool_segments(xr, lay.qb, lay.n_q, "seg")
            got = pool(x, lay.qb, lay.n_q, DIV_SEG).double().cpu().numpy()
            (assert_fp32_close if dtype == torch.float32 else assert_bf16_close)(got, ref, key + " qblock")


def test_pool_backward_broadcast():
    from llattn_amd import DIV_COUNT, DIV_SEG, pool
    dev = require_cuda()
    for T, seg, div in [(97, 17, DIV_COUNT), (61, 10, DIV_SEG), (2048, 128, DIV_COUNT)]:
        n = -(-T // seg)
        x = torch.randn(2, T, 16, device=dev, requires_grad=True)
        g = torch.randn(2, n, 16, device=dev)
        pool(x, seg, n, div).backward(g)
        cnt = np.array([min((i + 1) * seg, T) - i * seg for i in range(n)], dtype=np.float64)
        scale = 1.0 / cnt if div == DIV_COUNT else np.full(n, 1.0 / seg)
        ref = (g.double().cpu().numpy() * scale[None, :, None])[:, np.arange(T) // seg]
        assert_fp32_close(x.grad.double().cpu().numpy(), ref, f"T{T}")


# ---------------------------------------------------------------- BASELINE configs

def _c2_shape():
    return orc.BlockShape(d_model=1408, n_heads=16, window=64, local_block_size=256, latent_tokens=16,
                          latent_d_model=512, latent_heads=8)


def test_c2_bf16_batch_slices_match_fp32_reference():
    """Config 2 (0.55b layer, B16 T2048, bf16 autocast): out and dx of batch rows 0 and 15 vs the fp32
    torch CPU reference on those rows (rows are independent); weight grads at B=2 (same per-sequence shape)."""
    from oracle import torch_ref
    dev = require_cuda()
    shape = _c2_shape()
    torch.manual_seed(0)
    m = build_module(shape, None, dev)
    with torch.no_grad():
        for name, p in m.named_parameters():   # LocalLatentLM init (reference models.py:520-546), n_layers=22
            p.normal_(0.0, 0.02) if name.endswith("weight") else p.zero_()
            if name.startswith(("out.", "r_out.")) and name.endswith("weight"):
                p.mul_(1.0 / np.sqrt(44))
    x = torch.randn(16, 2048, 1408, device=dev).to(torch.bfloat16)
    dout = torch.randn(16, 2048, 1408, device=dev)
    _print_case("c2 full batch")
    out, dx, _ = run_module(m, x, dout, autocast_bf16=True)
    params = {n: p.detach().float().cpu() for n, p in m.named_parameters()}
    torch.set_num_threads(max(1, torch.get_num_threads()))
    for b in (0, 15):
        _print_case("c2 reference row", b)
        xb, db = x[b:b + 1].float().cpu(), dout[b:b + 1].float().cpu()
        o_ref, dx_ref, _ = torch_ref.block_forward_backward(params, xb, db, shape)
        assert_bf16_close(out[b:b + 1], o_ref.numpy(), f"out[{b}]")
        assert_bf16_close(dx[b:b + 1], dx_ref.numpy(), f"dx[{b}]")
        floor = reference_bf16_errors(params, xb, db, shape, {"out": o_ref.numpy(), "dx": dx_ref.numpy()})
        assert_within_floor(out[b:b + 1], o_ref.numpy(), floor["out"], f"out[{b}]")
        assert_within_floor(dx[b:b + 1], dx_ref.numpy(), floor["dx"], f"dx[{b}]")
    _print_case("c2 weight grads B=2")
    out2, dx2, g2 = run_module(m, x[:2], dout[:2], autocast_bf16=True)
    x2, d2 = x[:2].float().cpu(), dout[:2].float().cpu()
    _, _, g_ref = torch_ref.block_forward_backward(params, x2, d2, shape)
    floor = reference_bf16_errors(params, x2, d2, shape, {n: g_ref[n].numpy() for n in g_ref})
    for n in g_ref:
        assert_bf16_close(g2[n], g_ref[n].numpy(), n)
        assert_within_floor(g2[n], g_ref[n].numpy(), floor[n], n)


def test_c2_deterministic_and_finite():
    dev = require_cuda()
    _print_case("c2 determinism")
    shape = _c2_shape()
    torch.manual_seed(1)
    m = build_module(shape, None, dev)
    x = torch.randn(16, 2048, 1408, device=dev).to(torch.bfloat16)
    dout = torch.randn(16, 2048, 1408, device=dev)
    a = run_module(m, x, dout, autocast_bf16=True)
    b = run_module(m, x, dout, autocast_bf16=True)
    assert np.isfinite(a[0]).all() and np.isfinite(a[1]).all()
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])
    for n in a[2]:
        assert np.isfinite(a[2][n]).all(), n
        np.testing.assert_array_equal(a[2][n], b[2][n], err_msg=n)


def _config_row_check(cfg_name, rows):
    """Full-size BASELINE config on the GPU (bf16 autocast); rows of the batch vs the fp32 CPU reference."""
    from oracle import torch_ref
    dev = require_cuda()
    B, T, D, H, W, lbs, ntok, Ld, Lh, qbs = {
        "c3": (2, 16384, 1024, 16, 512, 256, 256, 64, 2, 0),
        "c4": (4, 8192, 1024, 16, 256, 256, 128, 64, 2, 64)}[cfg_name]
    shape = orc.BlockShape(d_model=D, n_heads=H, window=W, local_block_size=lbs, latent_tokens=ntok,
                           latent_d_model=Ld, latent_heads=Lh, latent_query_block_size=qbs)
    torch.manual_seed(3)
    m = build_module(shape, None, dev)
    with torch.no_grad():
        for name, p in m.named_parameters():
            p.normal_(0.0, 0.02) if name.endswith("weight") else p.normal_(0.0, 0.02)
    x = torch.randn(B, T, D, device=dev).to(torch.bfloat16)
    dout = torch.randn(B, T, D, device=dev)
    _print_case(cfg_name, "full batch")
    out, dx, grads = run_module(m, x, dout, autocast_bf16=True)
    params = {n: p.detach().float().cpu() for n, p in m.named_parameters()}
    del grads
    for b in rows:
        _print_case(cfg_name, "reference row", b)
        xb, db = x[b:b + 1].float().cpu(), dout[b:b + 1].float().cpu()
        o_ref, dx_ref, g_ref = torch_ref.block_forward_backward(params, xb, db, shape)
        assert_bf16_close(out[b:b + 1], o_ref.numpy(), f"out[{b}]")
        assert_bf16_close(dx[b:b + 1], dx_ref.numpy(), f"dx[{b}]")
        _print_case(cfg_name, "reference bf16 floor of row", b)
        floor = reference_bf16_errors(params, xb, db, shape, {"out": o_ref.numpy(), "dx": dx_ref.numpy(),
                                                               **{n: g_ref[n].numpy() for n in g_ref}})
        assert_within_floor(out[b:b + 1], o_ref.numpy(), floor["out"], f"out[{b}]")
        assert_within_floor(dx[b:b + 1], dx_ref.numpy(), floor["dx"], f"dx[{b}]")
        # every parameter gradient of that sequence alone (full T: the window > 64 two-pass local backward,
        # its gate partial rows, r_out's bias from dremote, the column-sum bias gradients of the D = 1024
        # projections, the macro-block scatter in config 4)
        _print_case(cfg_name, "parameter gradients of row", b)
        _, _, g_row = run_module(m, x[b:b + 1], dout[b:b + 1], autocast_bf16=True)
        assert set(g_row) == set(g_ref)
        for n in g_ref:
            assert_bf16_close(g_row[n], g_ref[n].numpy(), f"{n}[{b}]")
            assert_within_floor(g_row[n], g_ref[n].numpy(), floor[n], f"{n}[{b}]")
    return m, x, dout, params, shape


def test_c3_long_context_rows_match_fp32_reference():
    _config_row_check("c3", rows=(0, 1))


def test_c4_macro_block_rows_match_fp32_reference():
    _config_row_check("c4", rows=(0, 3))


def test_macro_block_equal_poolings_share_one_launch():
    """Macro-block mode with the latent chunk equal to the query block and T a multiple of it (config 4's
    64 / 64 at T = 8192): the query-block mean and the latent mean are the same values, so the forward pools
    x once.  Output and every gradient still match the fp32 reference, with the two poolings' gradients
    reaching x separately (reference models.py:159-230)."""
    from llattn_amd import ops
    from oracle import torch_ref
    dev = require_cuda()
    _print_case("shared pooling", "T 512, chunk 16, query block 16")
    shape = orc.BlockShape(d_model=256, n_heads=4, window=96, local_block_size=64, latent_tokens=32,
                           latent_d_model=128, latent_heads=2, latent_query_block_size=16)
    torch.manual_seed(5)
    m = build_module(shape, None, dev)
    with torch.no_grad():
        for p in m.parameters():
            p.normal_(0.0, 0.05)
    x = torch.randn(2, 512, 256, device=dev).to(torch.bfloat16)
    dout = torch.randn(2, 512, 256, device=dev)
    ops.EVENT_LOG = []
    try:
        out, dx, grads = run_module(m, x, dout, autocast_bf16=True)
        calls = [e[0] for e in ops.EVENT_LOG]
    finally:
        ops.EVENT_LOG = None
    # one in the forward (both poolings of x), one in the backward (dremote summed over each query block)
    assert calls.count("llattn_pool_fwd") == 2, calls
    params = {n: p.detach().float().cpu() for n, p in m.named_parameters()}
    o_ref, dx_ref, g_ref = torch_ref.block_forward_backward(params, x.float().cpu(), dout.float().cpu(), shape)
    assert_bf16_close(out, o_ref.numpy(), "out")
    assert_bf16_close(dx, dx_ref.numpy(), "dx")
    for n in g_ref:
        assert_bf16_close(grads[n], g_ref[n].numpy(), n)


# ---------------------------------------------------------------- profiling API (reference models.py:131-157)

PROFILE_KEYS = ("profile_local_latent_total_ms", "profile_qkv_ms", "profile_pool_ms", "profile_local_attention_ms",
                "profile_latent_attention_ms", "profile_gate_mix_ms", "profile_gate_mean", "profile_seq_len",
                "profile_local_block_size", "profile_latent_count", "profile_latent_chunk_size",
                "profile_latent_query_block_size")


@pytest.mark.parametrize("bf16", [False, True])
def test_profile_stats_on_config1(c1_golden, bf16):
    """set_profile(True) at the config-1 shape: the reference's twelve profile_* keys, averaged over forwards;
    positive stage times whose sum is the total (the gate mix runs inside the local kernel: 0 ms); the
    resolved sizes; gate_mean equal to the mean local gate weight w of the oracle's forward."""
    dev = require_cuda()
    _print_case("profile config 1", "bf16" if bf16 else "fp32")
    meta, params, x, dout, *_ = c1_golden
    shape = orc.BlockShape(d_model=256, n_heads=4, window=128, local_block_size=256, latent_tokens=8,
                           latent_d_model=32, latent_heads=2)
    m = build_module(shape, {k: v.numpy() for k, v in params.items()}, dev)
    assert m.get_profile_stats() == {}
    m.set_profile(True)
    xd = x.to(dev)
    for _ in range(3):
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16, enabled=bf16):
            m(xd)
    st = m.get_profile_stats()
    assert tuple(sorted(st)) == tuple(sorted(PROFILE_KEYS))
    for k in ("profile_qkv_ms", "profile_pool_ms", "profile_local_attention_ms", "profile_latent_attention_ms"):
        assert st[k] > 0.0, k
    assert st["profile_gate_mix_ms"] == 0.0
    parts = sum(st[k] for k in ("profile_qkv_ms", "profile_pool_ms", "profile_local_attention_ms",
                                "profile_latent_attention_ms", "profile_gate_mix_ms"))
    assert abs(st["profile_local_latent_total_ms"] - parts) < 1e-9
    assert st["profile_seq_len"] == 512 and st["profile_local_block_size"] == 256
    assert st["profile_latent_count"] == 8 and st["profile_latent_chunk_size"] == 64
    assert st["profile_latent_query_block_size"] == 1
    _, cache = orc.module_forward({k: v.double().numpy() for k, v in params.items()}, x.double().numpy(), shape,
                                  keep=True)
    assert abs(st["profile_gate_mean"] - float(np.mean(cache["w"]))) < (2e-3 if bf16 else 1e-5)
    m.set_profile(False)
    assert m.get_profile_stats() == {}


@pytest.mark.parametrize("cfg", ["c2_b2", "c2_b16", "macro"])
def test_split_head_qkv_matches_packed_layout(cfg, monkeypatch):
    """bf16 module forward + backward with the q|k|v|rq projection, r_out's output and the gradients of the
    latent output and of the core's output stored split-head (the default) against packed rows: only addresses
    differ, so the output and every gradient agree bit for bit."""
    import llattn_amd.module as mod
    import llattn_amd.ops as ops
    dev = require_cuda()
    if cfg.startswith("c2"):
        shape, B, T = _c2_shape(), int(cfg[4:]), 2048
    else:
        shape = orc.BlockShape(d_model=256, n_heads=4, window=96, local_block_size=64, latent_tokens=24,
                               latent_d_model=128, latent_heads=2, latent_query_block_size=16)
        B, T = 2, 520
    _print_case("split-head vs packed", cfg)
    torch.manual_seed(3)
    m = build_module(shape, None, dev)
    lay = m.layout(B, T)
    assert mod.heads_layout_ok(lay, shape.d_model, not lay.macro)
    x = torch.randn(B, T, shape.d_model, device=dev).to(torch.bfloat16)
    dout = torch.randn(B, T, shape.d_model, device=dev)
    a = run_module(m, x, dout, autocast_bf16=True)
    assert ops._remote_heads(lay, torch.bfloat16)
    assert ops._latent_grad_heads(lay) == (cfg == "c2_b16")
    assert mod.grad_heads_ok(B * T, shape.d_model, shape.d_model, lay.Dh) == (cfg == "c2_b16")
    monkeypatch.setattr(mod, "heads_layout_ok", lambda *args: False)
    monkeypatch.setattr(mod, "grad_heads_ok", lambda *args: False)
    monkeypatch.setattr(ops, "_remote_heads", lambda *args: False)
    monkeypatch.setattr(ops, "_latent_grad_heads", lambda *args: False)
    b = run_module(m, x, dout, autocast_bf16=True)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])
    for n in a[2]:
        np.testing.assert_array_equal(a[2][n], b[2][n], err_msg=n)
