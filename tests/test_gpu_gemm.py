"""GPU parity of the gfx950 projection GEMM (``llattn_gemm`` through the C ABI) against a float32 torch
product of the same bf16 operands.

Tolerances: bf16 output within 1e-2 of max(1, max|ref|) (one bf16 rounding of the result is 2^-8
relative); fp32 output within 1e-4 of max(1, max|ref|) (fp32 accumulation over up to 32k terms).
"""
from __future__ import annotations

import pytest
import torch

from gpu_helpers import require_cuda

pytestmark = pytest.mark.gpu

BF16_TOL, FP32_TOL = 1e-2, 1e-4


def _err(got, ref):
    return float((got.float() - ref).abs().max()) / max(1.0, float(ref.abs().max()))


def _rand(*shape, gen, dev):
    return torch.randn(*shape, device=dev, generator=gen).to(torch.bfloat16)


@pytest.mark.parametrize("M,N,K", [(256, 256, 64), (300, 264, 128), (97, 40, 192), (1000, 1408, 512),
                                   (32768, 4736, 1408)])
def test_linear_with_bias(M, N, K):
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: linear", M, N, K, flush=True)
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    x, w = _rand(M, K, gen=g, dev=dev), _rand(N, K, gen=g, dev=dev)
    b = torch.randn(N, device=dev, generator=g)
    ref = x.float() @ w.float().T + b
    assert _err(gemm.linear(x, w, b), ref) < BF16_TOL


@pytest.mark.parametrize("M,N,K,dt,acc", [(512, 64, 1024, torch.float32, False), (97, 40, 192, torch.float32, False),
                                          (512, 128, 1000, torch.float32, True), (512, 64, 1024, torch.bfloat16, True),
                                          (256, 1024, 1408, torch.bfloat16, False)])
def test_small_product_bias_and_accumulate(M, N, K, dt, acc):
    """Products of few 64 x 64 tiles over a long contraction (the pooled-latent and query-block projections)
    run as K splits plus the ordered reduction; bias and accumulation apply once, for an fp32 output too."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: small product", M, N, K, dt, acc, flush=True)
    g = torch.Generator(device=dev).manual_seed(M + 3 * N + K)
    x, w = _rand(M, K, gen=g, dev=dev), _rand(N, K, gen=g, dev=dev)
    b = torch.randn(N, device=dev, generator=g)
    c0 = torch.randn(M, N, device=dev, generator=g).to(dt)
    out = c0.clone() if acc else torch.empty((M, N), dtype=dt, device=dev)
    gemm.linear(x, w, b, out=out, accumulate=acc)
    ref = x.float() @ w.float().T + b + (c0.float() if acc else 0.0)
    assert _err(out, ref) < BF16_TOL


@pytest.mark.parametrize("M,N,K", [(1, 8, 8), (1, 40, 72), (97, 40, 200), (33, 264, 1000), (4096, 512, 200),
                                   (2000, 136, 8), (194, 208, 88)])
def test_linear_k_tail(M, N, K):
    """Contractions that are not a multiple of the 64-wide k step: the k-contiguous lanes past K read zero
    (a single row included, whose buffer ends inside the last step)."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: linear k tail", M, N, K, flush=True)
    g = torch.Generator(device=dev).manual_seed(M * 7 + N + K)
    # operands cut out of wider rows, so the elements past K are real data that must not leak in
    xb, wb = _rand(M, K + 24, gen=g, dev=dev) * 50, _rand(N, K + 24, gen=g, dev=dev) * 50
    x, w = xb[:, :K], wb[:, :K]
    b = torch.randn(N, device=dev, generator=g)
    assert _err(gemm.linear(x, w, b), x.float() @ w.float().T + b) < BF16_TOL


@pytest.mark.parametrize("M,N,K", [(32768, 1024, 64), (8192, 1408, 40), (32768, 256, 8)])
def test_linear_single_k_step(M, N, K):
    """A contraction of at most one 64-wide step on the persistent kernel (config 3's r_out forward, K = Ld =
    64): the pipeline runs it as two steps, the second reading zeros; the split-head store gives the same
    bits."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: linear single k step", M, N, K, flush=True)
    g = torch.Generator(device=dev).manual_seed(M + 5 * N + K)
    xb, wb = _rand(M, K + 24, gen=g, dev=dev), _rand(N, K + 24, gen=g, dev=dev)
    x, w = xb[:, :K], wb[:, :K]
    b = torch.randn(N, device=dev, generator=g)
    got = gemm.linear(x, w, b)
    assert _err(got, x.float() @ w.float().T + b) < BF16_TOL
    if N % 64 == 0:
        T = 2048
        heads = gemm.linear(x, w, b, heads=(T, 64, N // 64))
        assert torch.equal(heads, _to_heads(got, T, 64, N // 64))


@pytest.mark.parametrize("M,N,K", [(97, 40, 208), (300, 264, 1000), (3, 512, 72)])
def test_matmul_nn_k_tail(M, N, K):
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: nn k tail", M, N, K, flush=True)
    g = torch.Generator(device=dev).manual_seed(5 * M + N + K)
    ab = _rand(M, K + 40, gen=g, dev=dev) * 50
    a, b = ab[:, :K], _rand(K, N, gen=g, dev=dev)
    assert _err(gemm.matmul_nn(a, b), a.float() @ b.float()) < BF16_TOL


@pytest.mark.parametrize("K,M,N,S", [(194, 264, 136, 0), (33, 40, 96, 1), (1001, 1408, 512, 0), (5000, 264, 136, 3),
                                     (122, 16, 8, 2)])
def test_matmul_tn_token_tail(K, M, N, S):
    """Weight gradients over token counts that are not a multiple of 64 (nor of 8): rows past K lie beyond
    the operands' extent and read zero; with split-K the last split is the short one."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: tn token tail", K, M, N, S, flush=True)
    g = torch.Generator(device=dev).manual_seed(K + 3 * M + N)
    a, b = _rand(K, M, gen=g, dev=dev), _rand(K, N, gen=g, dev=dev)
    rs = torch.full((M,), float("nan"), device=dev)
    got = gemm.matmul_tn(a, b, split_k=S, rowsum=rs)
    assert _err(got, a.float().T @ b.float()) < FP32_TOL
    assert _err(rs, a.float().sum(0)) < FP32_TOL


@pytest.mark.parametrize("M,N,K", [(256, 256, 64), (300, 264, 128), (1000, 1408, 512)])
def test_matmul_nn(M, N, K):
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: nn", M, N, K, flush=True)
    g = torch.Generator(device=dev).manual_seed(7 * M + N)
    a, b = _rand(M, K, gen=g, dev=dev), _rand(K, N, gen=g, dev=dev)
    assert _err(gemm.matmul_nn(a, b), a.float() @ b.float()) < BF16_TOL


@pytest.mark.parametrize("B,T,N,K,pools", [
    (2, 300, 264, 128, [(64, 0)]),               # latent-style mean, last segment 44 tokens
    (3, 256, 136, 192, [(64, 1), (100, 0)]),     # query-block (zero-padded) mean and a ragged chunk mean
    (16, 2048, 1408, 4736, [(128, 0)]),          # config 2: qkv input gradient with the latent pooling
    (2, 97, 40, 64, [(17, 2)]),                  # plain sums
    (2, 2048, 1408, 4736, [(128, 0), (64, 1)]),  # a split-K shape: the addends join in the ordered reduction
])
def test_matmul_nn_rowadd(B, T, N, K, pools):
    """Input gradient with the pooling backward in its epilogue: a @ b + sum over poolings of rows[b, t // seg] /
    divisor (divisor 0: real tokens in the segment, 1: seg, 2: one), against fp32 torch; bf16 output."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: nn rowadd", B, T, N, K, pools, flush=True)
    g = torch.Generator(device=dev).manual_seed(B * T + N)
    a, b = _rand(B * T, K, gen=g, dev=dev), _rand(K, N, gen=g, dev=dev)
    ref = a.float() @ b.float()
    rowadd = []
    t = torch.arange(T, device=dev)
    for seg, div in pools:
        n_seg = -(-T // seg)
        rows = _rand(B * n_seg, N, gen=g, dev=dev) * 4
        s_id = t // seg
        count = torch.minimum((s_id + 1) * seg, torch.full_like(s_id, T)) - s_id * seg
        scale = {0: 1.0 / count.float(), 1: torch.full((T,), 1.0 / seg, device=dev), 2: torch.ones(T, device=dev)}[div]
        add = rows.float().view(B, n_seg, N)[:, s_id] * scale[None, :, None]
        ref = ref + add.reshape(B * T, N)
        rowadd.append((rows, T, seg, n_seg, div))
    assert _err(gemm.matmul_nn(a, b, rowadd=rowadd), ref) < BF16_TOL


@pytest.mark.parametrize("K,M,N,S", [(64, 256, 264, 1), (1024, 264, 136, 0), (2048, 40, 96, 1), (4096, 264, 136, 3),
                                     (4096, 1000, 520, 1), (32768, 1408, 1408, 0), (32768, 4736, 1408, 0),
                                     # N a multiple of 256 (no spare column): the first tile column's extra
                                     # products against ones; single pass, split-K, a ragged M and token tail
                                     (4096, 1000, 512, 1), (4096, 264, 256, 3), (1001, 520, 768, 2),
                                     (32768, 3200, 1024, 0), (32768, 1024, 1024, 0),
                                     # automatic 2-way splits of 90 tiles, a token tail in the last step, both
                                     # row-sum layouts
                                     (8200, 2304, 2504, 0), (8192, 2304, 2560, 0)])
def test_matmul_tn_rowsum(K, M, N, S):
    """Weight gradient with the bias gradient of the same pass: rowsum = a.sum(0), contracted against a column
    of ones in the spare column N of the last tile, or (N a multiple of 256) against ones in extra products of
    the first tile column; the product itself is unchanged by it."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: tn rowsum", K, M, N, S, flush=True)
    g = torch.Generator(device=dev).manual_seed(3 * K + M + N)
    a, b = _rand(K, M, gen=g, dev=dev), _rand(K, N, gen=g, dev=dev)
    rs = torch.full((M,), float("nan"), device=dev)
    got = gemm.matmul_tn(a, b, split_k=S, rowsum=rs)
    assert _err(got, a.float().T @ b.float()) < FP32_TOL
    assert _err(rs, a.float().sum(0)) < FP32_TOL
    # run to run: bitwise identical (ordered split-K reduction)
    rs2 = torch.empty_like(rs)
    got2 = gemm.matmul_tn(a, b, split_k=S, rowsum=rs2)
    assert torch.equal(rs, rs2) and torch.equal(got, got2)
    assert torch.equal(got, gemm.matmul_tn(a, b, split_k=S))  # the same products with and without the row sums


@pytest.mark.parametrize("K,M,N,S", [(64, 256, 256, 1), (1024, 264, 136, 0), (4096, 1408, 512, 4),
                                     (2048, 40, 96, 2), (4096, 264, 136, 3), (32768, 1408, 1408, 0),
                                     (32768, 4736, 1408, 0), (32768, 1408, 512, 0)])
def test_matmul_tn_fp32_out(K, M, N, S):
    """Weight-gradient products, including split-K (S > 1 or automatic) at the config-2 shapes."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: tn", K, M, N, S, flush=True)
    g = torch.Generator(device=dev).manual_seed(K + M)
    a, b = _rand(K, M, gen=g, dev=dev), _rand(K, N, gen=g, dev=dev)
    got = gemm.matmul_tn(a, b, split_k=S)
    assert got.dtype == torch.float32
    assert _err(got, a.float().T @ b.float()) < FP32_TOL


@pytest.mark.parametrize("M,N", [(1, 8), (97, 40), (1000, 136), (32768, 1408), (32768, 4736)])
def test_colsum(M, N):
    """Bias-gradient column sums, including ragged stripes and row blocks, and their determinism."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: colsum", M, N, flush=True)
    g = torch.Generator(device=dev).manual_seed(M + N)
    big = _rand(M, N + 16, gen=g, dev=dev)
    x = big[:, 8:8 + N]                       # strided view
    got = gemm.colsum(x)
    assert _err(got, x.float().sum(0)) < FP32_TOL
    torch.testing.assert_close(got, gemm.colsum(x), rtol=0, atol=0)


def test_accumulate_and_strided_views():
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: accumulate", flush=True)
    g = torch.Generator(device=dev).manual_seed(3)
    big = _rand(512, 200, gen=g, dev=dev)
    x = big[:, 8:136]                      # row stride 200, 128 columns
    w = _rand(256, 128, gen=g, dev=dev)
    c0 = _rand(512, 256, gen=g, dev=dev)
    out = c0.clone()
    gemm.linear(x, w, out=out, accumulate=True)
    assert _err(out, c0.float() + x.float() @ w.float().T) < BF16_TOL
    acc = torch.randn(256, 128, device=dev, generator=g)
    dy = _rand(1024, 256, gen=g, dev=dev)
    xx = _rand(1024, 128, gen=g, dev=dev)
    ref = acc + dy.float().T @ xx.float()
    gemm.matmul_tn(dy, xx, out=acc, accumulate=True)
    assert _err(acc, ref) < FP32_TOL


def test_deterministic_split_k():
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: split-K determinism", flush=True)
    g = torch.Generator(device=dev).manual_seed(11)
    a, b = _rand(32768, 512, gen=g, dev=dev), _rand(32768, 1408, gen=g, dev=dev)
    torch.testing.assert_close(gemm.matmul_tn(a, b), gemm.matmul_tn(a, b), rtol=0, atol=0)


def test_project_matches_fp32_linear():
    """The bf16 projection autograd function (shared-input layers in one GEMM) vs fp32 F.linear on the same
    bf16-rounded input: output, input gradient, fp32 weight and bias gradients."""
    from llattn_amd.linear import project
    dev = require_cuda()
    print("case: project", flush=True)
    torch.manual_seed(0)
    l1, l2 = torch.nn.Linear(256, 384).to(dev), torch.nn.Linear(256, 64).to(dev)
    x = torch.randn(2, 512, 256, device=dev).to(torch.bfloat16).requires_grad_(True)
    dy = torch.randn(2, 512, 448, device=dev)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        y = project(x, l1, l2)
    y.backward(dy.to(y.dtype))
    xr = x.detach().float().requires_grad_(True)
    # fp32 leaves holding the bf16-rounded weights, so the reference gradients are not rounded to bf16
    wr = torch.cat([l1.weight, l2.weight]).detach().to(torch.bfloat16).float().requires_grad_(True)
    br = torch.cat([l1.bias, l2.bias]).detach().to(torch.bfloat16).float().requires_grad_(True)
    yr = torch.nn.functional.linear(xr, wr, br)
    yr.backward(dy.to(torch.bfloat16).float())
    assert y.dtype == torch.bfloat16 and l1.weight.grad.dtype == torch.float32
    assert _err(y, yr) < BF16_TOL
    assert _err(x.grad, xr.grad) < BF16_TOL
    assert _err(torch.cat([l1.weight.grad, l2.weight.grad]), wr.grad) < 1e-3
    assert _err(torch.cat([l1.bias.grad, l2.bias.grad]), br.grad) < 1e-3


def test_project_with_pools_matches_fp32():
    """Poolings that ride on the projection: forward values and the input gradient, which sums the
    projection's and both poolings' gradients in place (ragged last segment in the second pooling)."""
    from llattn_amd import _lib as L
    from llattn_amd.linear import project
    dev = require_cuda()
    print("case: project+pools", flush=True)
    torch.manual_seed(1)
    lin = torch.nn.Linear(256, 320).to(dev)
    B, T, K = 2, 512, 256
    x = torch.randn(B, T, K, device=dev).to(torch.bfloat16).requires_grad_(True)
    pools = [(64, 8, L.DIV_COUNT), (100, 6, L.DIV_SEG)]
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        y, p1, p2 = project(x, lin, pools=pools)
    dy = torch.randn_like(y, dtype=torch.float32).to(torch.bfloat16)
    d1 = torch.randn_like(p1, dtype=torch.float32).to(torch.bfloat16)
    d2 = torch.randn_like(p2, dtype=torch.float32).to(torch.bfloat16)
    torch.autograd.backward([y, p1, p2], [dy, d1, d2])

    xr = x.detach().float().requires_grad_(True)
    wr = lin.weight.detach().to(torch.bfloat16).float()
    br = lin.bias.detach().to(torch.bfloat16).float()
    yr = torch.nn.functional.linear(xr, wr, br)
    r1 = xr.view(B, 8, 64, K).mean(2)
    pad = torch.nn.functional.pad(xr, (0, 0, 0, 600 - T))
    r2 = pad.view(B, 6, 100, K).sum(2) / 100
    torch.autograd.backward([yr, r1, r2], [dy.float(), d1.float(), d2.float()])
    assert _err(y, yr) < BF16_TOL
    assert _err(p1, r1) < BF16_TOL and _err(p2, r2) < BF16_TOL
    assert _err(x.grad, xr.grad) < BF16_TOL


@pytest.mark.parametrize("sizes", [[(4224, 1408), (512, 1408)], [(5,), (13,), (1029,)], [(7,)] * 11])
def test_pack_params_matches_torch_casts(sizes):
    """llattn_cast through pack_params: bf16 groups equal torch.cat(...).to(bfloat16) bit for bit (round to
    nearest even), fp32 groups equal the concatenation; lengths that are not multiples of 8 and more than 8
    arrays (two launches) included."""
    from llattn_amd.linear import pack_params
    dev = require_cuda()
    print("case: pack", sizes, flush=True)
    g = torch.Generator(device=dev).manual_seed(len(sizes))
    ts = [torch.randn(*s, device=dev, generator=g) * 3.0 for s in sizes]
    ts[0].view(-1)[:4] = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5e-39, float("inf")], device=dev)
    half = len(ts) // 2 or 1
    groups = [(ts[:half], torch.bfloat16)] + ([(ts[half:], torch.float32)] if ts[half:] else [])
    outs = pack_params(groups)
    assert torch.equal(outs[0].view(torch.int16), torch.cat(ts[:half]).to(torch.bfloat16).view(torch.int16))
    if ts[half:]:
        assert torch.equal(outs[1], torch.cat(ts[half:]))


@pytest.mark.parametrize("sizes", [
    [(4224, 1408), (512, 1408)],   # config 2's qkv | rq weights: two segments of one W^T
    [(1408, 512)],                 # r_out
    [(8, 72), (200, 72), (64, 72)],  # ragged 64-tiles, an 8-row segment
    [(12, 16)],                    # rows not a multiple of 8: no transposed copy
    [(64, 64)] * 9,                # more than 8 segments: two launches
])
def test_pack_params_transposed_copy(sizes):
    """llattn_cast_transposed through pack_params: the cast and its transposed copy equal torch's
    .to(bfloat16) and .t().contiguous() bit for bit, next to a plain bf16 group and an fp32 group in the same
    launch; with rows that are not multiples of 8 the pair carries None."""
    from llattn_amd.linear import pack_params
    dev = require_cuda()
    print("case: pack transposed", sizes, flush=True)
    g = torch.Generator(device=dev).manual_seed(7 + len(sizes))
    ts = [torch.randn(*s, device=dev, generator=g) * 3.0 for s in sizes]
    ts[0].view(-1)[:4] = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5e-39, float("inf")], device=dev)
    plain = [torch.randn(37, device=dev, generator=g)]
    bias = [torch.randn(24, device=dev, generator=g)]
    (w, w_t), wp, b = pack_params([(ts, torch.bfloat16, True), (plain, torch.bfloat16), (bias, torch.float32)])
    ref = torch.cat(ts).to(torch.bfloat16)
    assert torch.equal(w.view(torch.int16), ref.view(torch.int16))
    if all(s[0] % 8 == 0 and s[1] % 8 == 0 for s in sizes):
        assert w_t is not None and w_t.is_contiguous()
        assert torch.equal(w_t.view(torch.int16), ref.t().contiguous().view(torch.int16))
    else:
        assert w_t is None
    assert torch.equal(wp.view(torch.int16), plain[0].to(torch.bfloat16).view(torch.int16))
    assert torch.equal(b, bias[0])


def _gelu_and_grad(u):
    uu = u.float().requires_grad_(True)
    g = torch.nn.functional.gelu(uu)
    g.backward(torch.ones_like(g))
    return g.detach(), uu.grad


@pytest.mark.parametrize("M,N,K", [(32768, 4096, 1408), (300, 264, 200), (97, 40, 64)])
def test_linear_gelu_epilogue(M, N, K):
    """LLATTN_ACT_GELU: gelu and gelu' of the bf16-rounded pre-activation from one GEMM, against torch's F.gelu
    and its backward on the bf16-rounded fp32 product (small M takes the split-K reduction)."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: linear gelu", M, N, K, flush=True)
    g = torch.Generator(device=dev).manual_seed(M + 2 * N + K)
    x, w = _rand(M, K, gen=g, dev=dev), _rand(N, K, gen=g, dev=dev) * 0.1
    b = torch.randn(N, device=dev, generator=g) * 0.5
    got_g, got_gp = gemm.linear_gelu(x, w, b)
    ref_g, ref_gp = _gelu_and_grad((x.float() @ w.float().T + b).to(torch.bfloat16))
    for got, ref in ((got_g, ref_g), (got_gp, ref_gp)):
        assert got.dtype == torch.bfloat16
        assert _err(got, ref) < BF16_TOL
        # one bf16 rounding of the result, plus the rare pre-activation that rounds to the neighbouring bf16
        assert float((got.float() - ref).abs().mean()) < 2 ** -8 * float(ref.abs().mean())


@pytest.mark.parametrize("M,N,K", [(32768, 4096, 1408), (300, 264, 200), (97, 40, 64)])
def test_matmul_nn_scaled_epilogue(M, N, K):
    """LLATTN_ACT_MUL_AUX: bf16(dy W) * s elementwise, against torch on the bf16-rounded product."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: nn scaled", M, N, K, flush=True)
    g = torch.Generator(device=dev).manual_seed(3 * M + N + K)
    a, b = _rand(M, K, gen=g, dev=dev), _rand(K, N, gen=g, dev=dev) * 0.1
    sc = _rand(M, N, gen=g, dev=dev)
    got = gemm.matmul_nn_scaled(a, b, sc)
    ref = (a.float() @ b.float()).to(torch.bfloat16).float() * sc.float()
    assert _err(got, ref) < BF16_TOL


def test_feed_forward_matches_fp32_reference():
    """The LM's FeedForward under bf16 autocast (GELU in the GEMM epilogues) against fp32 w2(gelu(w1 x)) on the
    same bf16-rounded input and weights: output, input gradient, weight and bias gradients."""
    from llattn_amd.ffn import feed_forward
    dev = require_cuda()
    print("case: feed forward", flush=True)
    torch.manual_seed(2)
    w1, w2 = torch.nn.Linear(256, 1024).to(dev), torch.nn.Linear(1024, 256).to(dev)
    x = torch.randn(2, 300, 256, device=dev).to(torch.bfloat16).requires_grad_(True)
    dy = torch.randn(2, 300, 256, device=dev)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        y = feed_forward(x, w1, w2)
    y.backward(dy.to(y.dtype))
    xr = x.detach().float().requires_grad_(True)
    p = {n: t.detach().to(torch.bfloat16).float().requires_grad_(True)
         for n, t in (("w1", w1.weight), ("b1", w1.bias), ("w2", w2.weight), ("b2", w2.bias))}
    yr = torch.nn.functional.linear(torch.nn.functional.gelu(torch.nn.functional.linear(xr, p["w1"], p["b1"])),
                                    p["w2"], p["b2"])
    yr.backward(dy.to(torch.bfloat16).float())
    assert y.dtype == torch.bfloat16
    assert _err(y, yr) < BF16_TOL
    assert _err(x.grad, xr.grad) < BF16_TOL
    for got, name in ((w1.weight.grad, "w1"), (w1.bias.grad, "b1"), (w2.weight.grad, "w2"), (w2.bias.grad, "b2")):
        assert got.dtype == torch.float32
        assert _err(got, p[name].grad) < 2e-2, name


@pytest.mark.parametrize("R,C", [(1408, 1408), (4736, 1408), (8, 16), (200, 72)])
def test_transpose_bf16(R, C):
    """llattn_transpose is an exact copy: bitwise equal to torch's transpose (ragged 64-tiles included)."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: transpose", R, C, flush=True)
    g = torch.Generator(device=dev).manual_seed(R + C)
    w = _rand(R, C, gen=g, dev=dev)
    assert torch.equal(gemm.transpose(w), w.t().contiguous())


@pytest.mark.parametrize("M,N,K", [(32768, 1408, 1408), (32768, 512, 1408), (4096, 1408, 4096), (300, 264, 128)])
def test_input_grad_through_transposed_weight(M, N, K):
    """dy @ w through the persistent kernel and a transposed weight (large M) or the tiled kernel (small M)."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: input grad", M, N, K, flush=True)
    g = torch.Generator(device=dev).manual_seed(M + 3 * N + K)
    dy, w = _rand(M, K, gen=g, dev=dev), _rand(K, N, gen=g, dev=dev)
    assert _err(gemm.input_grad(dy, w), dy.float() @ w.float()) < BF16_TOL


@pytest.mark.parametrize("B,T,N,K,pools,bitwise", [
    (16, 2048, 1408, 4736, [(128, 0)], True),          # config 2: the qkv input gradient with the latent pooling
    (4, 2000, 520, 264, [(64, 0), (100, 1)], True),    # ragged segments, two addends, K with a 64-wide tail
    (2, 4096, 136, 1024, [(512, 2)], False),           # 32 tiles: the tiled kernel splits K here
])
def test_input_grad_rowadd_persistent_equals_tiled(B, T, N, K, pools, bitwise):
    """The input gradient with pooled-gradient row addends through the transposed weight and the persistent
    kernel matches fp32 torch, and gives the same bits as the tiled kernel with transposing fragment reads
    wherever that one does not split K (same k order, same epilogue arithmetic)."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: input grad rowadd persistent", B, T, N, K, pools, flush=True)
    g = torch.Generator(device=dev).manual_seed(B * T + N + K)
    dy, w = _rand(B * T, K, gen=g, dev=dev), _rand(K, N, gen=g, dev=dev)
    ref = dy.float() @ w.float()
    rowadd = []
    t = torch.arange(T, device=dev)
    for seg, div in pools:
        n_seg = -(-T // seg)
        rows = _rand(B * n_seg, N, gen=g, dev=dev) * 4
        s_id = t // seg
        count = torch.minimum((s_id + 1) * seg, torch.full_like(s_id, T)) - s_id * seg
        scale = {0: 1.0 / count.float(), 1: torch.full((T,), 1.0 / seg, device=dev), 2: torch.ones(T, device=dev)}[div]
        ref = ref + (rows.float().view(B, n_seg, N)[:, s_id] * scale[None, :, None]).reshape(B * T, N)
        rowadd.append((rows, T, seg, n_seg, div))
    got = gemm.input_grad(dy, w, rowadd=rowadd)
    if bitwise:
        assert torch.equal(got, gemm.matmul_nn(dy, w, rowadd=rowadd))
    assert _err(got, ref) < BF16_TOL


# ---- split-head operands (llattn_heads_layout): the q|k|v projection output stored as head slabs ----

def _to_heads(x: torch.Tensor, T: int, dh: int, n: int, tdh: int = 0) -> torch.Tensor:
    """Row-major [B T, W] -> the same matrix in split-head storage, as a [B T, W] tensor: the first n dh
    columns as [B][n][T][dh] slabs, then the other columns packed [B T][W - n dh] (tdh = 0) or as
    [B][(W - n dh) / tdh][T][tdh] slabs (torch permute, independent of the kernels' offset arithmetic)."""
    R, W = x.shape
    B, c = R // T, n * dh
    head = x[:, :c].reshape(B, T, n, dh).permute(0, 2, 1, 3).reshape(-1)
    rest = x[:, c:]
    if tdh:
        rest = rest.reshape(B, T, (W - c) // tdh, tdh).permute(0, 2, 1, 3)
    return torch.cat([head, rest.reshape(-1)]).view(R, W)


def _from_heads(s: torch.Tensor, T: int, dh: int, n: int, tdh: int = 0) -> torch.Tensor:
    R, W = s.shape
    B, c = R // T, n * dh
    flat = s.reshape(-1)
    head = flat[:R * c].view(B, n, T, dh).permute(0, 2, 1, 3).reshape(R, c)
    rest = flat[R * c:]
    rest = rest.view(B, (W - c) // tdh, T, tdh).permute(0, 2, 1, 3).reshape(R, W - c) if tdh else rest.view(R, W - c)
    return torch.cat([head, rest], dim=1)


HEADS_CASES = [  # (B, T, dh, n, tail, K, tdh): head columns n dh, plus `tail` columns (packed, or as slabs of tdh
    # columns); K the contraction
    (2, 160, 32, 6, 64, 192, 0),
    (3, 97, 88, 12, 0, 136, 0),      # T not a multiple of 32 or 256: slabs start inside tiles and k steps
    (2, 300, 16, 6, 512, 256, 0),
    (1, 64, 64, 3, 8, 72, 0),
    (16, 2048, 88, 48, 512, 1408, 0),  # config 2's q|k|v|rq with the latent queries packed
    (2, 160, 32, 6, 64, 192, 16),
    (3, 97, 88, 12, 96, 136, 24),    # tail slabs that start inside tiles, heads not a multiple of 16 wide
    (2, 300, 16, 6, 512, 256, 64),
    (16, 2048, 88, 48, 512, 1408, 64),  # config 2: q|k|v|rq of the 0.55b layer
    (16, 2048, 64, 8, 0, 1408, 0),   # config 2: the latent output's gradient as Lh slabs
]


@pytest.mark.parametrize("case", HEADS_CASES)
def test_linear_split_head_output(case):
    """The persistent kernel's stores in split-head order: the same product as the row-major output."""
    from llattn_amd import gemm
    B, T, dh, n, tail, K, tdh = case
    dev = require_cuda()
    print("case: linear split-head C", case, flush=True)
    g = torch.Generator(device=dev).manual_seed(B * T + dh + n + tail + tdh)
    M, N = B * T, n * dh + tail
    x, w = _rand(M, K, gen=g, dev=dev), _rand(N, K, gen=g, dev=dev)
    b = torch.randn(N, device=dev, generator=g)
    got = gemm.linear(x, w, b, heads=(T, dh, n, tdh))
    assert _err(_from_heads(got, T, dh, n, tdh), x.float() @ w.float().T + b) < BF16_TOL
    if M * N >= 1 << 24:  # both on the persistent kernel: only the store order differs
        assert torch.equal(got, _to_heads(gemm.linear(x, w, b), T, dh, n, tdh))


def test_input_grad_split_head_output():
    """The input gradient on the persistent kernel stored as head slabs (the latent output's gradient of
    config 2, [B][Lh][n_q][Ldh]): the same bits as the row-major input gradient (256 output tiles: unsplit on
    the persistent kernel too), permuted; the small-M route refuses a split-head output."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: input_grad split-head", flush=True)
    g = torch.Generator(device=dev).manual_seed(5)
    B, T, Lh, Ldh, D = 16, 2048, 8, 64, 1408
    dy, w = _rand(B * T, D, gen=g, dev=dev), _rand(D, Lh * Ldh, gen=g, dev=dev)
    plain = gemm.input_grad(dy, w)
    got = gemm.input_grad(dy, w, heads=(T, Ldh, Lh))
    assert torch.equal(got, _to_heads(plain, T, Ldh, Lh))
    assert _err(plain, dy.float() @ w.float()) < BF16_TOL
    with pytest.raises(ValueError, match="persistent"):
        gemm.input_grad(dy[:1024], w, heads=(1024, Ldh, Lh))


@pytest.mark.parametrize("M,N,K", [(1, 8, 1), (97, 40, 64), (64, 64, 16), (300, 264, 1000), (33, 130, 37),
                                   (2048, 1408, 256), (256, 1024, 1408)])
def test_gemm_f32_products(M, N, K):
    """The fp32 products of llattn_gemm_f32 against float64 CPU references: x W^T + b, dy W (through a strided
    view of W), dy^T x with the row sums of dy^T (the bias gradient), and accumulation into C; ragged tiles
    and contraction lengths that are not multiples of 4 or 16 included."""
    from llattn_amd import gemm
    dev = require_cuda()
    print("case: gemm f32", M, N, K, flush=True)
    g = torch.Generator(device=dev).manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, device=dev, generator=g)
    w_full = torch.randn(N, K + 8, device=dev, generator=g)
    w = w_full[:, :K]  # leading dimension K + 8
    b = torch.randn(N, device=dev, generator=g)
    ref = (x.double() @ w.double().T + b.double()).float()
    assert _err(gemm.linear_f32(x, w, b), ref) < 1e-5
    dy = torch.randn(M, N, device=dev, generator=g)
    assert _err(gemm.matmul_nn_f32(dy, w), (dy.double() @ w.double()).float()) < 1e-5
    rs = torch.full((N,), float("nan"), device=dev)
    dw = gemm.matmul_tn_f32(dy, x, rowsum=rs)
    assert _err(dw, (dy.double().T @ x.double()).float()) < 1e-5
    assert _err(rs, dy.double().sum(0).float()) < 1e-5
    assert torch.equal(dw, gemm.matmul_tn_f32(dy, x))  # the same products with and without the row sums
    out = torch.randn(M, N, device=dev, generator=g)
    ref_acc = out.double() + x.double() @ w.double().T
    gemm._run_f32(M, N, K, x, False, w, False, out, accumulate=True)
    assert _err(out, ref_acc.float()) < 1e-5

