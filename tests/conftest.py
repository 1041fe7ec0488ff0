"""Shared test setup: the ``gpu`` marker, import paths and golden-fixture loaders."""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
PKG_ROOT = REPO / "local-latent-attention_amd"
GOLDEN = REPO / "tests" / "golden"

for p in (str(REPO), str(PKG_ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def pytest_sessionfinish(session, exitstatus):
    """With LLATTN_PARITY_LOG set, write every GPU parity comparison (raw and scaled errors, the bar used) as
    JSON lines to that file."""
    import os
    path = os.environ.get("LLATTN_PARITY_LOG")
    if not path or "gpu_helpers" not in sys.modules:
        return
    with open(path, "w") as f:
        for row in sys.modules["gpu_helpers"].RECORD:
            f.write(json.dumps(row) + "\n")


E2E_CASES = ("tiny_tok", "tiny_macro", "w1_chunk1", "dh88_single_block", "qbs1_is_tokenwise", "macro_ragged")


def load_case(name: str):
    """Return (shape_kwargs, B, T, x, dout, params, out, dx, grads) of a golden end-to-end case."""
    z = np.load(GOLDEN / f"case_{name}.npz", allow_pickle=False)
    meta = json.loads(str(z["meta"]))
    params = {k[2:]: z[k] for k in z.files if k.startswith("p:")}
    grads = {k[2:]: z[k] for k in z.files if k.startswith("g:")}
    return meta, z["x"], z["dout"], params, z["out"], z["dx"], grads


def shape_from_meta(meta):
    from oracle.llattn_oracle import BlockShape
    return BlockShape(d_model=meta["d_model"], n_heads=meta["n_heads"], window=meta["local_window"],
                      local_block_size=meta["local_block_size"], latent_tokens=meta["latent_tokens"],
                      latent_d_model=meta["latent_d_model"], latent_heads=meta["latent_heads"],
                      latent_query_block_size=meta["latent_query_block_size"])


def c1_inputs():
    """Regenerate BASELINE config 1 inputs exactly as ``tests/golden/make_golden.py`` drew them:
    ``torch.manual_seed(0)``; the block's Linear layers in ``LocalLatentAttention.__init__``
    order with torch default init; then x, then dout."""
    import torch
    import torch.nn as nn
    torch.manual_seed(0)
    D, Ld, Dh = 256, 32, 64
    layers = [("qkv_proj", nn.Linear(D, 3 * D)), ("rq_proj", nn.Linear(D, Ld)), ("rkv_proj", nn.Linear(D, 2 * Ld)),
              ("r_out", nn.Linear(Ld, D)), ("out", nn.Linear(D, D)),
              ("gate_local", nn.Linear(Dh, 1, bias=False)), ("gate_remote", nn.Linear(Dh, 1, bias=False))]
    params = {}
    for name, lin in layers:
        params[name + ".weight"] = lin.weight.detach().clone()
        if lin.bias is not None:
            params[name + ".bias"] = lin.bias.detach().clone()
    x = torch.randn(2, 512, 256)
    dout = torch.randn(2, 512, 256)
    return params, x, dout


@pytest.fixture(scope="session")
def c1_golden():
    z = np.load(GOLDEN / "case_c1.npz", allow_pickle=False)
    meta = json.loads(str(z["meta"]))
    params, x, dout = c1_inputs()
    sums = meta["input_sums"]
    assert abs(float(x.double().sum()) - sums["x"]) < 1e-6
    assert abs(float(dout.double().sum()) - sums["dout"]) < 1e-6
    for n, p in params.items():
        assert abs(float(p.double().sum()) - sums["p:" + n]) < 1e-6, n
    grads = {k[2:]: z[k] for k in z.files if k.startswith("g:")}
    return meta, params, x, dout, z["out"], z["dx"], grads
