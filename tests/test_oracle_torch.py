"""Pins of the torch CPU restatement (``oracle/torch_ref.py``) -- CPU only."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import E2E_CASES, load_case, shape_from_meta
from oracle import llattn_oracle as orc
from oracle import torch_ref


@pytest.mark.parametrize("name", E2E_CASES)
def test_torch_ref_matches_reference_golden(name):
    meta, x, dout, params, out_ref, dx_ref, grads_ref = load_case(name)
    shape = shape_from_meta(meta)
    pt = {k: torch.from_numpy(v) for k, v in params.items()}
    out, dx, grads = torch_ref.block_forward_backward(pt, torch.from_numpy(x), torch.from_numpy(dout), shape)
    np.testing.assert_allclose(out.numpy(), out_ref, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dx.numpy(), dx_ref, rtol=1e-8, atol=1e-10)
    for n in grads_ref:
        np.testing.assert_allclose(grads[n].numpy(), grads_ref[n], rtol=1e-8, atol=1e-9, err_msg=n)


def test_torch_ref_config1_fp32(c1_golden):
    meta, params, x, dout, out_ref, dx_ref, grads_ref = c1_golden
    shape = orc.BlockShape(d_model=256, n_heads=4, window=128, local_block_size=256, latent_tokens=8,
                           latent_d_model=32, latent_heads=2)
    out, dx, grads = torch_ref.block_forward_backward(params, x, dout, shape)
    assert float((out.numpy() - out_ref).__abs__().max()) < 1e-5
    assert float((dx.numpy() - dx_ref).__abs__().max()) < 1e-5
    for n in grads_ref:
        scale = max(1.0, float(np.abs(grads_ref[n]).max()))
        assert float(np.abs(grads[n].numpy() - grads_ref[n]).max()) < 1e-5 * scale, n


@pytest.mark.parametrize("qbs", [0, 64])
def test_torch_ref_matches_numpy_oracle_long(qbs):
    """A shape the golden cases do not cover: several local blocks, W < bs, T % chunk != 0."""
    shape = orc.BlockShape(d_model=64, n_heads=2, window=24, local_block_size=64, latent_tokens=9,
                           latent_d_model=32, latent_heads=2, latent_query_block_size=qbs)
    rng = np.random.default_rng(3)
    params = orc.init_params(shape, rng, std=0.3)
    x = rng.standard_normal((2, 300, 64))
    dout = rng.standard_normal((2, 300, 64))
    out, cache = orc.module_forward(params, x, shape, keep=True)
    dx, grads = orc.module_backward(params, x, shape, cache, dout)
    pt = {k: torch.from_numpy(v) for k, v in params.items()}
    o2, dx2, g2 = torch_ref.block_forward_backward(pt, torch.from_numpy(x), torch.from_numpy(dout), shape)
    np.testing.assert_allclose(o2.numpy(), out, rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(dx2.numpy(), dx, rtol=1e-8, atol=1e-9)
    for n in grads:
        np.testing.assert_allclose(g2[n].numpy(), grads[n], rtol=1e-8, atol=1e-9, err_msg=n)
