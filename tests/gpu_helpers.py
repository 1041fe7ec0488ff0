"""Helpers shared by the GPU parity tests."""
from __future__ import annotations

import numpy as np
import torch

from oracle.llattn_oracle import BlockShape

FP32_TOL = 1e-4            # max-abs, fp32 kernels vs the float64 / fp32 reference
BF16_MAX_TOL = 2e-2        # max-abs, bf16 kernels vs the fp32 reference
BF16_MEANREL_TOL = 1e-2    # mean(|a-b|) / mean(|b|)


# Every comparison made through assert_fp32_close / assert_bf16_close, as
# (case, tensor, dtype bar, raw max|a-ref|, max|ref|, scaled max-abs, mean-rel, max-abs bar, mean-rel bar);
# conftest writes it out when LLATTN_PARITY_LOG names a file.
RECORD: list = []
CASE = [""]


def set_case(name: str) -> None:
    CASE[0] = name


def _record(what, a, ref, bar, tmx, tmr):
    a = np.asarray(a, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    mx, mr = err_stats(a, ref)
    RECORD.append({"case": CASE[0], "tensor": what, "bar": bar, "raw_max_abs": float(np.abs(a - ref).max()),
                   "max_ref": float(np.abs(ref).max()), "scaled_max_abs": mx, "mean_rel": mr,
                   "max_abs_bar": tmx, "mean_rel_bar": tmr})
    return mx, mr


def require_cuda():
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return torch.device("cuda:0")


def build_module(shape: BlockShape, params: dict | None = None, device="cuda:0", dtype=torch.float32):
    from llattn_amd import LocalLatentAttentionTriton
    m = LocalLatentAttentionTriton(shape.d_model, shape.n_heads, shape.latent_heads, shape.latent_d_model,
                                   shape.latent_tokens, shape.window, local_block_size=shape.local_block_size,
                                   latent_query_block_size=shape.latent_query_block_size)
    if params is not None:
        sd = {k: torch.as_tensor(np.asarray(v)).to(torch.float32) for k, v in params.items()}
        m.load_state_dict(sd)
    return m.to(device=device, dtype=dtype)


def run_module(m, x: torch.Tensor, dout: torch.Tensor, autocast_bf16: bool = False):
    x = x.detach().clone().requires_grad_(True)
    for p in m.parameters():
        p.grad = None
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16, enabled=autocast_bf16):
        out = m(x)
    out.backward(dout.to(out.dtype))
    grads = {n: p.grad.detach().float().cpu().double().numpy() for n, p in m.named_parameters()}
    return out.detach().float().cpu().double().numpy(), x.grad.detach().float().cpu().double().numpy(), grads


def err_stats(a, ref):
    """(max|a-ref| / max(1, max|ref|), mean|a-ref| / mean|ref|).  The mean-relative term is 0 when the
    reference is zero to rounding (e.g. dQ with a single key per query, where the softmax is saturated):
    a relative error of an exact zero carries no information, and the max-abs term still bounds it."""
    a = np.asarray(a, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    d = np.abs(a - ref)
    scale = max(1.0, float(np.abs(ref).max()))
    mref = float(np.abs(ref).mean())
    mean_rel = float(d.mean() / mref) if mref > 1e-9 * scale else 0.0
    return float(d.max()) / scale, mean_rel


def assert_fp32_close(a, ref, what=""):
    mx, _ = _record(what, a, ref, "fp32", FP32_TOL, None)
    assert mx <= FP32_TOL, f"{what}: scaled max-abs {mx:.3e} > {FP32_TOL}"


def assert_bf16_close(a, ref, what="", floor=None):
    """bf16 bar: scaled max-abs <= 2e-2 and mean-rel <= 1e-2.  With ``floor`` = the (max, mean-rel) error
    that the reference math itself reaches when run under bf16 autocast on the same inputs, the bar is
    raised to twice that floor where the floor alone already exceeds it."""
    tmx, tmr = BF16_MAX_TOL, BF16_MEANREL_TOL
    if floor is not None:
        tmx, tmr = max(tmx, 2.0 * floor[0]), max(tmr, 2.0 * floor[1])
    mx, mr = _record(what, a, ref, "bf16" if floor is None else "bf16 floor", tmx, tmr)
    assert mx <= tmx, f"{what}: scaled max-abs {mx:.3e} > {tmx:.3e}"
    assert mr <= tmr, f"{what}: mean-rel {mr:.3e} > {tmr:.3e}"


def reference_bf16_errors(params: dict, x: torch.Tensor, dout: torch.Tensor, shape, refs: dict) -> dict:
    """Raw max|a - ref| that the reference math itself (the fp32 torch CPU restatement, oracle/torch_ref.py)
    reaches when run under CPU bf16 autocast on the same weights and inputs, for every tensor of ``refs``
    (keys ``out``, ``dx`` and parameter names, fp32 reference values): the bf16 floor of a full-size row."""
    from oracle import torch_ref
    with torch.autocast("cpu", dtype=torch.bfloat16):
        o, dx, g = torch_ref.block_forward_backward(params, x, dout, shape)
    got = {"out": o, "dx": dx, **g}
    return {k: float(np.abs(got[k].detach().double().numpy() - np.asarray(refs[k], dtype=np.float64)).max())
            for k in refs}


FLOOR_RAW_TOL = 2e-2  # raw max-abs below which no floor is needed


def assert_within_floor(a, ref, floor_raw: float, what=""):
    """Where the raw max-abs of a bf16 result exceeds 2e-2 (large tensors such as bias gradients summed over
    16k-32k tokens, whose bf16 ulp alone is above it), it must stay within twice the error the reference's
    own math reaches under bf16 autocast on the same inputs (:func:`reference_bf16_errors`)."""
    raw = float(np.abs(np.asarray(a, dtype=np.float64) - np.asarray(ref, dtype=np.float64)).max())
    RECORD.append({"case": CASE[0], "tensor": what, "bar": "raw vs bf16 floor", "raw_max_abs": raw,
                   "floor_raw_max_abs": floor_raw, "raw_bar": max(FLOOR_RAW_TOL, 2.0 * floor_raw)})
    if raw > FLOOR_RAW_TOL:
        assert raw <= 2.0 * floor_raw, f"{what}: raw max-abs {raw:.3e} > 2 x reference bf16 floor {floor_raw:.3e}"


def bf16_floor(params: dict, x_bf16: np.ndarray, dout: np.ndarray, shape, grads_ref: dict) -> dict:
    """Per-parameter (max, mean-rel) error of the reference math (torch CPU restatement) under
    bf16 autocast against the float64 golden gradients: the precision a bf16 run can be expected to reach."""
    from oracle import torch_ref
    p = {k: torch.tensor(np.asarray(v), dtype=torch.float32) for k, v in params.items()}
    with torch.autocast("cpu", dtype=torch.bfloat16):
        _, _, g = torch_ref.block_forward_backward(p, torch.tensor(x_bf16, dtype=torch.float32),
                                                   torch.tensor(dout, dtype=torch.float32), shape)
    return {n: err_stats(g[n].float().numpy(), grads_ref[n]) for n in grads_ref}
