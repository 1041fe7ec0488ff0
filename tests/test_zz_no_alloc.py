"""llattn_local_gate_bwd_noalloc (the backward with the library's own scratch) against
llattn_local_gate_bwd (caller workspace), both called through the C ABI on the same inputs.

The two run the same kernels in the same order, so their outputs must be bitwise equal.  Each case
makes two calls in a row, the second on a smaller input, so the second reads scratch that still holds
the first call's partial sums.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from gpu_helpers import require_cuda

pytestmark = pytest.mark.gpu

_byref = ctypes.byref


def _inputs(L, B, T, H, Dh, W, block, dtype, per_head, seed, device):
    """Random q|k|v (packed as the qkv projection writes them), remote rows, gates and dy; o_local, lse
    and w from llattn_local_gate_fwd, as the backward receives them."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    D = H * Dh
    qkv = torch.randn((B, T, 3 * D), generator=g).to(device=device, dtype=dtype)
    remote = torch.randn((B, T, D), generator=g).to(device=device, dtype=dtype)
    gshape = (H, Dh) if per_head else (Dh,)
    gl = (0.3 * torch.randn(gshape, generator=g)).to(device).contiguous()
    gr = (0.3 * torch.randn(gshape, generator=g)).to(device).contiguous()
    dy = torch.randn((B, T, D), generator=g).to(device=device, dtype=dtype)
    lay = L.Layout(B, T, H, Dh, 1, 16, W, block, T, 1, 1, T)
    shape = lay.shape(dtype, per_head)
    sb, sn = qkv.stride(0), qkv.stride(1)
    q, k, v = (L.view(qkv, sb, sn, Dh, i * D) for i in range(3))
    rem = L.view(remote, remote.stride(0), remote.stride(1), Dh)
    y = torch.empty((B, T, H, Dh), dtype=dtype, device=device)
    ol = torch.empty_like(y)
    lse = torch.empty((B, H, T), dtype=torch.float32, device=device)
    w = torch.empty_like(lse)
    lib = L.load()
    L.check(lib.llattn_local_gate_fwd(_byref(shape), _byref(q), _byref(k), _byref(v), _byref(rem), gl.data_ptr(),
                                      gr.data_ptr(), _byref(L.view_bnhd(y)), _byref(L.view_bnhd(ol)), lse.data_ptr(),
                                      w.data_ptr(), L.stream_ptr(device)), "llattn_local_gate_fwd")
    keep = (qkv, remote, gl, gr, dy, ol, lse, w)
    return shape, (q, k, v, rem), keep


def _backward(L, shape, views, keep, noalloc, device):
    q, k, v, rem = views
    qkv, remote, gl, gr, dy, ol, lse, w = keep
    B, T, H, Dh = shape.B, shape.T, shape.H, shape.Dh
    dt = qkv.dtype
    outs = [torch.full((B, T, H, Dh), float("nan"), dtype=dt, device=device) for _ in range(4)]
    ng = (H, Dh) if shape.gate_per_head else (Dh,)
    dgl = torch.full(ng, float("nan"), device=device)
    dgr = torch.full(ng, float("nan"), device=device)
    dbr = torch.full((H * Dh,), float("nan"), device=device)
    lib = L.load()
    args = [_byref(shape), _byref(q), _byref(k), _byref(v), _byref(rem), gl.data_ptr(), gr.data_ptr(),
            _byref(L.view_bnhd(ol)), lse.data_ptr(), w.data_ptr(), _byref(L.view(dy, dy.stride(0), dy.stride(1), Dh)),
            *[_byref(L.view_bnhd(o)) for o in outs], dgl.data_ptr(), dgr.data_ptr(), dbr.data_ptr()]
    if noalloc:
        rc = lib.llattn_local_gate_bwd_noalloc(*args, L.stream_ptr(device))
        L.check(rc, "llattn_local_gate_bwd_noalloc")
    else:
        nws = L.workspace_bytes(shape, L.WS_LOCAL_BWD)
        ws = torch.empty((nws,), dtype=torch.uint8, device=device)
        rc = lib.llattn_local_gate_bwd(*args, ws.data_ptr(), nws, L.stream_ptr(device))
        L.check(rc, "llattn_local_gate_bwd")
    torch.cuda.synchronize(device)
    return [*outs, dgl, dgr, dbr]


def test_noalloc_backward_under_graph_capture():
    """The entry point's first call of the process made inside HIP graph capture (torch.cuda.graph): the
    per-device scratch address is looked up there.  The captured graph is replayed three times, with eager
    kernels and synchronizations between the replays, and every replay matches the workspace backward bit
    for bit.  Defined first in this file so that no earlier test has called the entry point."""
    from llattn_amd import _lib as L
    dev = require_cuda()
    B, T, H, Dh, W, block, dt = 2, 1024, 16, 88, 64, 256, torch.bfloat16
    print(f"noalloc graph capture: B={B} T={T} H={H} Dh={Dh} W={W} {dt}", flush=True)
    shape, views, keep = _inputs(L, B, T, H, Dh, W, block, dt, False, seed=23, device=dev)
    ref = _backward(L, shape, views, keep, noalloc=False, device=dev)
    q, k, v, rem = views
    qkv, remote, gl, gr, dy, ol, lse, w = keep
    outs = [torch.full((B, T, H, Dh), float("nan"), dtype=dt, device=dev) for _ in range(4)]
    dgl, dgr = torch.full((Dh,), float("nan"), device=dev), torch.full((Dh,), float("nan"), device=dev)
    dbr = torch.full((H * Dh,), float("nan"), device=dev)
    args = [_byref(shape), _byref(q), _byref(k), _byref(v), _byref(rem), gl.data_ptr(), gr.data_ptr(),
            _byref(L.view_bnhd(ol)), lse.data_ptr(), w.data_ptr(), _byref(L.view(dy, dy.stride(0), dy.stride(1), Dh)),
            *[_byref(L.view_bnhd(o)) for o in outs], dgl.data_ptr(), dgr.data_ptr(), dbr.data_ptr()]
    lib = L.load()
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.llattn_local_gate_bwd_noalloc(*args, L.stream_ptr(dev))
    L.check(rc, "llattn_local_gate_bwd_noalloc (captured)")
    for rep in range(3):
        for o in (*outs, dgl, dgr, dbr):
            o.fill_(float("nan"))
        _backward(L, shape, views, keep, noalloc=False, device=dev)  # eager work between the replays
        graph.replay()
        torch.cuda.synchronize(dev)
        for j, (a, b) in enumerate(zip([*outs, dgl, dgr, dbr], ref)):
            assert torch.equal(a, b), f"replay {rep} output {j}: max diff {(a.float() - b.float()).abs().max().item()}"


# (B, T, H, Dh, W, block, dtype, per_head): a large call, then a smaller one on the same path
CASES = [
    ("bf16 fused (config-2 heads)", [(4, 2048, 16, 88, 64, 256, torch.bfloat16, False),
                                     (2, 640, 16, 88, 64, 256, torch.bfloat16, False)]),
    ("fp32 two-kernel (config-1 heads)", [(2, 512, 4, 64, 128, 256, torch.float32, False),
                                          (1, 300, 4, 64, 128, 256, torch.float32, True)]),
    ("bf16 two-kernel (window > 64)", [(1, 1024, 8, 64, 256, 256, torch.bfloat16, True),
                                       (1, 200, 8, 64, 96, 128, torch.bfloat16, False)]),
]


@pytest.mark.parametrize("name,calls", CASES, ids=[c[0] for c in CASES])
def test_noalloc_backward_equals_workspace_backward(name, calls):
    from llattn_amd import _lib as L
    dev = require_cuda()
    for i, (B, T, H, Dh, W, block, dt, per_head) in enumerate(calls):
        print(f"noalloc case {name!r} call {i}: B={B} T={T} H={H} Dh={Dh} W={W} block={block} {dt}", flush=True)
        shape, views, keep = _inputs(L, B, T, H, Dh, W, block, dt, per_head, seed=17 + i, device=dev)
        ref = _backward(L, shape, views, keep, noalloc=False, device=dev)
        got = _backward(L, shape, views, keep, noalloc=True, device=dev)
        for j, (a, b) in enumerate(zip(got, ref)):
            assert torch.isfinite(b).all(), f"call {i} output {j}: reference not finite"
            assert torch.equal(a, b), f"call {i} output {j}: max diff {(a.float() - b.float()).abs().max().item()}"


def test_noalloc_backward_rejects_shapes_beyond_its_scratch():
    from llattn_amd import _lib as L
    dev = require_cuda()
    # bf16, window 512: the two-kernel backward needs dO_local (B*T*H*Dh bf16 = 16 MiB here) in scratch
    shape, views, keep = _inputs(L, 1, 8192, 16, 64, 512, 512, torch.bfloat16, False, seed=5, device=dev)
    with pytest.raises(RuntimeError, match="scratch bytes"):
        _backward(L, shape, views, keep, noalloc=True, device=dev)
