"""Pins of the CPU oracle (``oracle/llattn_oracle.py``) -- CPU only.

Each test checks the oracle against something other than its own formula:
the reference's golden vectors, a brute-force replay of the reference's
procedure, a closed form, or finite differences.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import E2E_CASES, GOLDEN, load_case, shape_from_meta
from oracle import llattn_oracle as orc


# ---------------------------------------------------------------- key set

def _oracle_mask(T, W, lbs):
    lay = orc.seq_layout(orc.BlockShape(d_model=8, n_heads=1, window=W, local_block_size=lbs), T)
    j = np.arange(T)
    return (j[None, :] >= lay.key_lo[:, None]) & (j[None, :] <= lay.key_hi[:, None])


def _replay_block_loop(T, W, lbs):
    """Brute force of the reference procedure: per query block, the key slice
    [max(0,q0-W+1), q_end) and the distance mask 0 < i-j <= W (models.py:249-292)."""
    bs = min(T, max(W, lbs))
    allowed = np.zeros((T, T), dtype=bool)
    for q0 in range(0, T, bs):
        q1 = min(q0 + bs, T)
        k0 = max(0, q0 - W + 1)
        for i in range(q0, q1):
            for j in range(k0, q1):
                if 0 < i - j <= W:
                    allowed[i, j] = True
    return allowed


def test_keyset_matches_reference_golden():
    z = np.load(GOLDEN / "keyset.npz")
    assert len(z.files) >= 7
    for key in z.files:
        T, W, bs = (int(t[1:]) if t[0] == "T" or t[0] == "W" else int(t[2:]) for t in key.split("_"))
        ref = np.unpackbits(z[key], axis=1, count=T).astype(bool)
        np.testing.assert_array_equal(_oracle_mask(T, W, bs), ref, err_msg=key)


@pytest.mark.parametrize("T,W,lbs", [(97, 16, 32), (300, 64, 256), (64, 1, 8), (257, 128, 100), (40, 3, 3),
                                     (513, 200, 64), (1, 1, 1), (2, 5, 1)])
def test_keyset_matches_block_loop_replay(T, W, lbs):
    np.testing.assert_array_equal(_oracle_mask(T, W, lbs), _replay_block_loop(T, W, lbs))


def test_block_start_quirk_counts():
    # with bs = 256, W = 64 the query at each block start i >= W loses its farthest key
    m = _oracle_mask(2048, 64, 256)
    counts = m.sum(1)
    for i in range(2048):
        expect = min(i, 64) - (1 if (i % 256 == 0 and i >= 64) else 0)
        assert counts[i] == expect, i
    assert counts.sum() == sum(min(i, 64) for i in range(2048)) - 7   # 7 keys lost per sequence


# ---------------------------------------------------------------- pooling

def test_pooling_matches_reference_golden():
    z = np.load(GOLDEN / "pool.npz")
    keys = sorted({k.rsplit("_", 1)[0] for k in z.files})
    assert len(keys) >= 10
    for key in keys:
        T, ntok, qbs = (int(t[1:]) for t in key.split("_"))
        shape = orc.BlockShape(d_model=4, n_heads=1, window=4, latent_tokens=ntok, latent_query_block_size=qbs)
        lay = orc.seq_layout(shape, T)
        x = z[key + "_x"]
        np.testing.assert_allclose(orc.pool_segments(x, lay.chunk, lay.n_chunks, "count"), z[key + "_pooled"],
                                   rtol=1e-12, atol=1e-12, err_msg=key)
        np.testing.assert_array_equal(lay.chunk_ids, z[key + "_ids"], err_msg=key)
        if qbs > 1:
            np.testing.assert_allclose(orc.pool_segments(x, lay.qb, lay.n_q, "seg"), z[key + "_qpooled"],
                                       rtol=1e-12, atol=1e-12, err_msg=key)
            np.testing.assert_array_equal(lay.q_chunk_ids, z[key + "_qids"], err_msg=key)


@pytest.mark.parametrize("T,ntok", [(97, 6), (130, 128), (7, 16), (2048, 16), (16384, 256), (1, 1)])
def test_pooling_closed_form(T, ntok):
    rng = np.random.default_rng(T)
    x = rng.standard_normal((1, T, 3))
    lay = orc.seq_layout(orc.BlockShape(d_model=3, n_heads=1, window=4, latent_tokens=ntok), T)
    assert lay.n_chunks <= ntok and lay.n_chunks == len(np.unique(lay.chunk_ids))
    pooled = orc.pool_segments(x, lay.chunk, lay.n_chunks, "count")
    for n in range(lay.n_chunks):
        np.testing.assert_allclose(pooled[0, n], x[0, lay.chunk_ids == n].mean(0), rtol=1e-12)


# ---------------------------------------------------------------- attention pieces

def _dense_masked_attention(q, k, v, mask):
    """Brute force: per query, an explicit softmax over its allowed keys (python loop)."""
    B, H, T, Dh = q.shape
    out = np.zeros_like(q)
    for b in range(B):
        for h in range(H):
            for i in range(T):
                js = np.nonzero(mask[i])[0]
                if len(js) == 0:
                    continue
                s = np.array([q[b, h, i] @ k[b, h, j] for j in js]) / math.sqrt(Dh)
                p = np.exp(s - s.max())
                p /= p.sum()
                out[b, h, i] = sum(pj * v[b, h, j] for pj, j in zip(p, js))
    return out


@pytest.mark.parametrize("T,W,lbs", [(70, 9, 16), (40, 1, 8), (33, 64, 256)])
def test_banded_local_attention_matches_brute_force(T, W, lbs):
    rng = np.random.default_rng(1)
    q, k, v = (rng.standard_normal((1, 2, T, 8)) for _ in range(3))
    lay = orc.seq_layout(orc.BlockShape(d_model=16, n_heads=2, window=W, local_block_size=lbs), T)
    O, LSE = orc.local_attention(q, k, v, lay, qblk=16)
    np.testing.assert_allclose(O, _dense_masked_attention(q, k, v, _oracle_mask(T, W, lbs)), rtol=1e-10, atol=1e-12)
    empty = lay.key_lo > lay.key_hi
    assert np.all(np.isneginf(LSE[..., empty])) and np.all(np.isfinite(LSE[..., ~empty]))


def test_full_window_is_strictly_causal_attention():
    """W >= T and bs >= T: every query sees exactly its strict past (a causal mask shifted by one)."""
    T = 45
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal((2, 1, T, 4)) for _ in range(3))
    lay = orc.seq_layout(orc.BlockShape(d_model=4, n_heads=1, window=T, local_block_size=T), T)
    O, _ = orc.local_attention(q, k, v, lay)
    strict = np.tril(np.ones((T, T), dtype=bool), k=-1)
    np.testing.assert_allclose(O, _dense_masked_attention(q, k, v, strict), rtol=1e-10, atol=1e-12)
    assert np.all(O[:, :, 0] == 0)


def test_latent_attention_chunk1_is_strictly_causal():
    rng = np.random.default_rng(3)
    T = 30
    rq, gk, gv = (rng.standard_normal((1, 2, T, 4)) for _ in range(3))
    L, P = orc.latent_attention(rq, gk, gv, np.arange(T))
    strict = np.tril(np.ones((T, T), dtype=bool), k=-1)
    np.testing.assert_allclose(L, _dense_masked_attention(rq, gk, gv, strict), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(P.sum(-1)[..., 1:], 1.0, rtol=1e-12)
    assert np.all(L[:, :, 0] == 0)


def test_gate_identities():
    rng = np.random.default_rng(4)
    O, R = rng.standard_normal((2, 1, 2, 5, 6))
    gl, gr = rng.standard_normal((2, 6))
    Y, w, s_l, s_r = orc.gate_mix(O, R, gl, gr)
    np.testing.assert_allclose(w, 1.0 / (1.0 + np.exp(-(s_l - s_r))), rtol=1e-12)
    # zero gate weights mix the branches half and half
    Y1, w1, _, _ = orc.gate_mix(O, R, np.zeros(6), np.zeros(6))
    np.testing.assert_allclose(w1, 0.5)
    np.testing.assert_allclose(Y1, 0.5 * (O + R), rtol=1e-12)
    # saturating the gate gives the pure branches
    big = 1e4
    Yl, wl, _, _ = orc.gate_mix(np.ones_like(O), R, np.full(6, big), np.zeros(6))
    np.testing.assert_allclose(Yl, np.ones_like(O), rtol=1e-12)
    Yr, wr, _, _ = orc.gate_mix(np.ones_like(O), R, np.full(6, -big), np.zeros(6))
    np.testing.assert_allclose(Yr, R, rtol=1e-12)


# ---------------------------------------------------------------- end to end

@pytest.mark.parametrize("name", E2E_CASES)
def test_module_forward_backward_match_reference_golden(name):
    meta, x, dout, params, out_ref, dx_ref, grads_ref = load_case(name)
    shape = shape_from_meta(meta)
    out, cache = orc.module_forward(params, x, shape, keep=True)
    np.testing.assert_allclose(out, out_ref, rtol=1e-9, atol=1e-11)
    dx, grads = orc.module_backward(params, x, shape, cache, dout)
    np.testing.assert_allclose(dx, dx_ref, rtol=1e-9, atol=1e-10)
    assert set(grads) == set(grads_ref)
    for n in grads:
        np.testing.assert_allclose(grads[n], grads_ref[n], rtol=1e-8, atol=1e-9, err_msg=n)


def test_chunk0_tokens_get_r_out_bias():
    meta, x, dout, params, *_ = load_case("tiny_tok")
    shape = shape_from_meta(meta)
    _, cache = orc.module_forward(params, x, shape, keep=True)
    lay = cache["lay"]
    chunk0 = lay.q_chunk_ids == 0
    R = cache["R_q"]
    np.testing.assert_allclose(R[:, chunk0], np.broadcast_to(params["r_out.bias"], R[:, chunk0].shape), rtol=1e-12)


def test_config1_matches_reference_golden(c1_golden):
    meta, params_t, x_t, dout_t, out_ref, dx_ref, grads_ref = c1_golden
    shape = orc.BlockShape(d_model=256, n_heads=4, window=128, local_block_size=256, latent_tokens=8,
                           latent_d_model=32, latent_heads=2)
    params = {k: v.double().numpy() for k, v in params_t.items()}
    x = x_t.double().numpy()
    out, cache = orc.module_forward(params, x, shape, keep=True)
    np.testing.assert_allclose(out, out_ref, atol=2e-5, rtol=0)
    dx, grads = orc.module_backward(params, x, shape, cache, dout_t.double().numpy())
    np.testing.assert_allclose(dx, dx_ref, atol=2e-5, rtol=0)
    for n in grads:
        scale = max(1.0, float(np.abs(grads_ref[n]).max()))
        np.testing.assert_allclose(grads[n], grads_ref[n], atol=2e-5 * scale, rtol=0, err_msg=n)


@pytest.mark.parametrize("qbs", [0, 5])
def test_backward_matches_finite_differences(qbs):
    shape = orc.BlockShape(d_model=12, n_heads=2, window=4, local_block_size=6, latent_tokens=4,
                           latent_d_model=8, latent_heads=2, latent_query_block_size=qbs)
    rng = np.random.default_rng(7 + qbs)
    params = orc.init_params(shape, rng, std=0.4)
    x = rng.standard_normal((2, 13, 12))
    dout = rng.standard_normal((2, 13, 12))
    out, cache = orc.module_forward(params, x, shape, keep=True)
    dx, grads = orc.module_backward(params, x, shape, cache, dout)

    def f():
        return float((orc.module_forward(params, x, shape) * dout).sum())

    eps = 1e-6
    checks = [("x", x, dx)] + [(n, params[n], grads[n]) for n in orc.PARAM_NAMES]
    for name, arr, g in checks:
        flat = arr.reshape(-1)
        idx = rng.choice(flat.size, size=min(flat.size, 12), replace=False)
        for i in idx:
            old = flat[i]
            flat[i] = old + eps
            fp = f()
            flat[i] = old - eps
            fm = f()
            flat[i] = old
            num = (fp - fm) / (2 * eps)
            assert abs(num - g.reshape(-1)[i]) < 1e-6 * max(1.0, abs(num)), (name, i, num, g.reshape(-1)[i])
