"""kda_chunkwise_bwd_noalloc (the backward without a caller workspace, on the
library's static scratch buffer) against kda_chunkwise_bwd (workspace from the
torch allocator), through the C ABI: two calls in a row, the second with a
smaller shape, each must give bit-identical gradients -- the same kernels run
on the same inputs, only the workspace address differs.  The second call
reuses the buffer the first one left behind (the kernels write every
workspace element before reading it)."""

from __future__ import annotations

import ctypes
import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def native(kda_pkg):
    mod = importlib.import_module("kimi_linear_amd._native")
    mod.load()
    return mod


def _inputs(kda_pkg, B, T, H, K, V, dtype, seed):
    wl = importlib.import_module("kimi_linear_amd.workloads")
    inp = wl.make_inputs(B, T, H, K, V, seed=seed, qkv_dtype=dtype, state_std=0.02)
    q, k, v = (inp[n].to(DEV).contiguous() for n in ("q", "k", "v"))
    g, beta = inp["g"].to(DEV).float().contiguous(), inp["beta"].to(DEV).float().contiguous()
    s0 = inp["state"].to(DEV)
    kda = importlib.import_module("kimi_linear_amd.kda")
    with torch.no_grad():
        _, _, ckpt = kda._forward("chunkwise", q, k, v, g, beta, s0, T, torch.float32, ckpt=True)
    gen = torch.Generator(device=DEV).manual_seed(seed + 1)
    d_o = torch.randn(B, T, H, V, device=DEV, generator=gen).to(dtype)
    d_s = torch.randn(B, H, K, V, device=DEV, generator=gen)
    return dict(q=q, k=k, v=v, g=g, beta=beta, ckpt=ckpt, d_o=d_o, d_s=d_s)


def _run(native, entry, x, B, T, H, K, V, dtype, workspace):
    outs = dict(dq=torch.empty(B, T, H, K, device=DEV, dtype=dtype),
                dk=torch.empty(B, T, H, K, device=DEV, dtype=dtype),
                dv=torch.empty(B, T, H, V, device=DEV, dtype=dtype),
                dg=torch.empty(B, T, H, K, device=DEV),
                dbeta=torch.empty(B, T, H, device=DEV),
                ds0=torch.empty(B, H, K, V, device=DEV))
    codes = {torch.float32: native.DTYPE_F32, torch.float16: native.DTYPE_F16, torch.bfloat16: native.DTYPE_BF16}
    a = native.KdaBwdArgs()
    a.B, a.T, a.H, a.K, a.V = B, T, H, K, V
    a.q, a.k, a.v, a.g, a.beta = (x[n].data_ptr() for n in ("q", "k", "v", "g", "beta"))
    a.ckpt, a.d_o, a.d_state_out = x["ckpt"].data_ptr(), x["d_o"].data_ptr(), x["d_s"].data_ptr()
    a.dq, a.dk, a.dg = outs["dq"].data_ptr(), outs["dk"].data_ptr(), outs["dg"].data_ptr()
    a.dbeta, a.dv, a.d_state_in = outs["dbeta"].data_ptr(), outs["dv"].data_ptr(), outs["ds0"].data_ptr()
    a.workspace = workspace.data_ptr() if workspace is not None else None
    a.scale = float(K) ** -0.5
    a.io_dtype = codes[dtype]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    status = getattr(native.load(), entry)(ctypes.byref(a), stream)
    assert status == native.STATUS_OK, native.status_str(status)
    return outs


def test_noalloc_backward_equals_workspace_backward(kda_pkg, native):
    lib = native.load()
    # first a larger call, then a smaller one on the buffer the first left behind
    for (B, T, H, K, V, dtype) in [(2, 200, 4, 128, 128, torch.float16), (1, 70, 2, 64, 64, torch.float32)]:
        print(f"no-alloc backward B={B} T={T} H={H} K={K} V={V} {dtype}", flush=True)
        need = lib.kda_chunkwise_bwd_workspace_size(B, T, H, K, V)
        assert 0 < need <= native.BWD_SCRATCH_BYTES
        x = _inputs(kda_pkg, B, T, H, K, V, dtype, seed=B * 1000 + T)
        ws = torch.empty(need, device=DEV, dtype=torch.uint8)
        ref = _run(native, "kda_chunkwise_bwd", x, B, T, H, K, V, dtype, ws)
        got = _run(native, "kda_chunkwise_bwd_noalloc", x, B, T, H, K, V, dtype, None)
        torch.cuda.synchronize()
        for name in ref:
            assert torch.isfinite(ref[name]).all(), name
            assert torch.equal(got[name], ref[name]), name


def test_noalloc_backward_under_graph_capture(kda_pkg, native):
    """The entry is for callers that capture their work: after an eager call on
    the device (which resolves the scratch address), a captured call replays
    to the eager gradients three times, with other eager work on the same
    buffers in between."""
    B, T, H, K, V, dtype = 1, 96, 4, 128, 128, torch.float16
    print(f"no-alloc backward under capture B={B} T={T} H={H} K={K} V={V} {dtype}", flush=True)
    x = _inputs(kda_pkg, B, T, H, K, V, dtype, seed=77)
    eager = _run(native, "kda_chunkwise_bwd_noalloc", x, B, T, H, K, V, dtype, None)
    torch.cuda.synchronize()
    holder = {}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _run(native, "kda_chunkwise_bwd_noalloc", x, B, T, H, K, V, dtype, None)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        holder["outs"] = _run(native, "kda_chunkwise_bwd_noalloc", x, B, T, H, K, V, dtype, None)
    outs = holder["outs"]
    for rep in range(3):
        for t in outs.values():
            t.fill_(float("nan"))
        # eager work on the shared scratch between replays (a smaller shape)
        y = _inputs(kda_pkg, 1, 40, 2, 64, 64, torch.float32, seed=78 + rep)
        _run(native, "kda_chunkwise_bwd_noalloc", y, 1, 40, 2, 64, 64, torch.float32, None)
        graph.replay()
        torch.cuda.synchronize()
        for name in eager:
            assert torch.equal(outs[name], eager[name]), (rep, name)
    del graph
