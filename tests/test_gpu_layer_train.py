"""GPU parity of the layer's training path: the native backward kernels of the
pre-processing (conv, SiLU, L2 norm, gates) and of the output epilogue, and
the gradients of the whole layer, against autograd of the fp64 oracle on the
CPU (the oracle's forward is pinned by the reference fixtures; its gradient
is autograd's).

Tolerances, relative L2 error of each gradient: fp32 inputs 1e-4 for the
kernels (2e-4 for the layer: its fp32 core checkpoints are exact and the
parameter gradients sum over every token; measured <= 6e-5), fp16 1e-3 for the
kernels (measured <= 2.9e-4) and 2e-3 for the layer (measured <= 9.1e-4), bf16
6e-3 (measured <= 2.4e-3) and 1.5e-2 (measured <= 6.7e-3): the 16-bit paths
round every activation, and the upstream gradients, to 11 or 8 bits.
"""

from __future__ import annotations

import pytest
import torch

from oracle.kda_layer_oracle import (gates_ref, head_rmsnorm_ref, kda_layer_ref, l2norm_ref, make_layer_params,
                                     short_conv_ref)

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL_K = {torch.float32: 1e-4, torch.float16: 1e-3, torch.bfloat16: 6e-3}
TOL_L = {torch.float32: 2e-4, torch.float16: 2e-3, torch.bfloat16: 1.5e-2}


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp(min=1e-300)).item()


def _prep_inputs(B, T, H, K, V, cs, dtype, seed, bias=True, tiny=False):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    Dk, Dv = H * K, H * V
    xs = [r(B, T, D) for D in (Dk, Dk, Dv)]
    if tiny:
        # q rows far below eps: the L2 norm's clamp is active
        xs[0] = xs[0] * 1e-9
    ws = [0.5 * r(D, 1, cs) for D in (Dk, Dk, Dv)]
    bs = [0.1 * r(D) if bias else None for D in (Dk, Dk, Dv)]
    gk = r(B, T, Dk)
    logit = r(B, T, H)
    a_log = torch.rand(H, K, generator=gen) * 2.0
    dt_bias = 0.5 * r(H, K)
    inp = dict(x=[x.to(dtype) for x in xs], w=ws, b=bs, gk=gk.to(dtype), logit=logit.to(dtype), a_log=a_log,
               dt_bias=dt_bias)
    up = dict(dq=r(B, T, H, K), dk=r(B, T, H, K), dv=r(B, T, H, V), dg=r(B, T, H, K), dbeta=r(B, T, H))
    return inp, up


def _prep_ref(inp, H, K, V, eps):
    """fp64 autograd reference of kda_prep (kda.py:399-461 without the cache)."""
    xs = [x.double().requires_grad_() for x in inp["x"]]
    ws = [w.double().requires_grad_() for w in inp["w"]]
    bs = [b.double().requires_grad_() if b is not None else None for b in inp["b"]]
    gk = inp["gk"].double().requires_grad_()
    logit = inp["logit"].double().requires_grad_()
    a_log = inp["a_log"].double().requires_grad_()
    dt_bias = inp["dt_bias"].double().requires_grad_()
    B, T = xs[0].shape[:2]
    c = [short_conv_ref(x, w, b) for x, w, b in zip(xs, ws, bs)]
    silu = lambda u: u * torch.sigmoid(u)  # noqa: E731
    q = l2norm_ref(silu(c[0]).view(B, T, H, K), eps)
    k = l2norm_ref(silu(c[1]).view(B, T, H, K), eps)
    v = silu(c[2]).view(B, T, H, V)
    g, beta = gates_ref(gk.view(B, T, H, K), logit, a_log, dt_bias)
    leaves = dict(x=xs, w=ws, b=bs, gk=gk, logit=logit, a_log=a_log, dt_bias=dt_bias)
    return (q, k, v, g, beta), leaves


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K,V,T,cs,bias", [(64, 64, 100, 4, True), (128, 64, 16, 4, False), (64, 128, 70, 2, True),
                                           (128, 128, 129, 3, True)])
def test_prep_backward_vs_autograd(kda_pkg, dtype, K, V, T, cs, bias):
    """Ragged T (tiles of 64 and steps of 16 cut mid-way), conv sizes 2-4,
    with and without conv bias."""
    import importlib
    ops = importlib.import_module("kimi_linear_amd.layer_ops")
    B, H, eps = 2, 2, 1e-6
    inp, up = _prep_inputs(B, T, H, K, V, cs, dtype, seed=3 + K + T, bias=bias)
    dev = lambda t: t.to(DEV).requires_grad_() if t is not None else None  # noqa: E731
    xs = [dev(x) for x in inp["x"]]
    ws = [dev(w.to(dtype)) for w in inp["w"]]
    bs = [dev(b.to(dtype)) if b is not None else None for b in inp["b"]]
    gk, logit = dev(inp["gk"]), dev(inp["logit"])
    a_log, dt_bias = dev(inp["a_log"]), dev(inp["dt_bias"])
    outs = ops.kda_prep_train(*xs, ws, bs, gk, a_log, dt_bias, logit, num_heads=H, head_dim=K, value_head_dim=V,
                              l2_eps=eps)
    ups = [up[n] for n in ("dq", "dk", "dv", "dg", "dbeta")]
    torch.autograd.backward(outs, [u.to(DEV).to(o.dtype) for u, o in zip(ups, outs)])
    # the reference sees the parameters as the kernels do (16-bit conv weights)
    inp_ref = dict(inp, w=[w.to(dtype) for w in inp["w"]], b=[b.to(dtype) if b is not None else None for b in inp["b"]])
    ref_out, leaves = _prep_ref(inp_ref, H, K, V, eps)
    # upstream gradients as the kernels receive them (rounded to the output dtype)
    torch.autograd.backward(ref_out, [u.to(o.dtype).double() if i < 3 else u.double()
                                      for i, (u, o) in enumerate(zip(ups, outs))])
    errs = {}
    for i, n in enumerate("qkv"):
        errs[f"d{n}_in"] = rel(xs[i].grad, leaves["x"][i].grad)
        errs[f"dw_{n}"] = rel(ws[i].grad, leaves["w"][i].grad)
        if bias:
            errs[f"db_{n}"] = rel(bs[i].grad, leaves["b"][i].grad)
    errs["dgk"] = rel(gk.grad, leaves["gk"].grad)
    errs["dlogit"] = rel(logit.grad, leaves["logit"].grad)
    errs["dA_log"] = rel(a_log.grad, leaves["a_log"].grad)
    errs["ddt_bias"] = rel(dt_bias.grad, leaves["dt_bias"].grad)
    worst = max(errs, key=errs.get)
    print(f"prep backward {dtype} K={K} V={V} T={T} cs={cs} bias={bias}: worst {worst} {errs[worst]:.2e}", flush=True)
    assert errs[worst] <= TOL_K[dtype], errs


def test_prep_backward_l2_clamp(kda_pkg):
    """q rows with sum of squares below eps^2: y = s / eps, so ds = dy / eps
    (the clamp's branch), as autograd of the clamped reference gives."""
    import importlib
    ops = importlib.import_module("kimi_linear_amd.layer_ops")
    B, T, H, K, V, cs, eps = 1, 32, 2, 64, 64, 4, 1e-3
    inp, up = _prep_inputs(B, T, H, K, V, cs, torch.float32, seed=11, tiny=True)
    xs = [x.to(DEV).requires_grad_() for x in inp["x"]]
    ws = [w.to(DEV) for w in inp["w"]]
    bs = [torch.zeros_like(b).to(DEV) for b in inp["b"]]
    outs = ops.kda_prep_train(*xs, ws, bs, inp["gk"].to(DEV), inp["a_log"].to(DEV), inp["dt_bias"].to(DEV),
                              inp["logit"].to(DEV), num_heads=H, head_dim=K, value_head_dim=V, l2_eps=eps)
    ups = [up[n] for n in ("dq", "dk", "dv", "dg", "dbeta")]
    torch.autograd.backward(outs[:3], [u.to(DEV) for u in ups[:3]])
    inp_ref = dict(inp, b=[torch.zeros_like(b) for b in inp["b"]])
    ref_out, leaves = _prep_ref(inp_ref, H, K, V, eps)
    torch.autograd.backward(ref_out[:3], [u.double() for u in ups[:3]])
    e = rel(xs[0].grad, leaves["x"][0].grad)
    print(f"prep backward, clamped L2 norm: dq_in rel {e:.2e}", flush=True)
    assert e <= 1e-4


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("V,T", [(64, 40), (128, 33), (128, 8)])
def test_output_backward_vs_autograd(kda_pkg, dtype, V, T):
    import importlib
    ops = importlib.import_module("kimi_linear_amd.layer_ops")
    B, H, eps = 2, 3, 1e-5
    gen = torch.Generator().manual_seed(V + T)
    o = torch.randn(B, T, H, V, generator=gen).to(dtype)
    gate = torch.randn(B, T, H * V, generator=gen).to(dtype)
    w = 1 + 0.1 * torch.randn(H, V, generator=gen)
    dy = torch.randn(B, T, H * V, generator=gen).to(dtype)
    od, gd, wd = (t.to(DEV).requires_grad_() for t in (o, gate, w))
    y = ops.kda_output_train(od, gd, wd, eps)
    y.backward(dy.to(DEV))
    o64, g64, w64 = (t.double().requires_grad_() for t in (o, gate, w))
    n = head_rmsnorm_ref(o64, w64, eps)
    yr = (n * torch.sigmoid(g64.view(B, T, H, V))).reshape(B, T, H * V)
    yr.backward(dy.double())
    errs = {"do": rel(od.grad, o64.grad), "dgate": rel(gd.grad, g64.grad), "dweight": rel(wd.grad, w64.grad)}
    worst = max(errs, key=errs.get)
    print(f"output backward {dtype} V={V} T={T}: worst {worst} {errs[worst]:.2e}", flush=True)
    assert errs[worst] <= TOL_K[dtype], errs


def _layer(kda_pkg, dtype, seed, **kw):
    cfg = kda_pkg.linear_attn_config(**{"hidden_size": 256, "num_heads": 2, "gate_low_rank": 64,
                                        "output_gate_low_rank": 64, **kw})
    m = kda_pkg.KimiDeltaAttention(cfg)
    m.load_state_dict(make_layer_params(cfg, seed=seed))
    return m.to(device=DEV, dtype=dtype), cfg


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("T,hd", [(64, 128), (100, 64), (40, 128)])
def test_layer_training_gradients_vs_oracle(kda_pkg, dtype, T, hd):
    """Every parameter's gradient and x's, for T a multiple of the chunk
    size, ragged T (the reference's chunkwise body + recurrent tail) and
    T < chunk_size."""
    m, cfg = _layer(kda_pkg, dtype, seed=5, head_dim=hd, value_head_dim=hd)
    B = 2
    gen = torch.Generator().manual_seed(T + hd)
    x = torch.randn(B, T, 256, generator=gen).to(dtype)
    wout = torch.randn(B, T, 256, generator=gen)
    xd = x.to(DEV).requires_grad_()
    out = m(xd)
    (out.float() * wout.to(DEV)).sum().backward()
    p64 = {n: t.detach().double().cpu().requires_grad_() for n, t in m.state_dict().items()}
    x64 = x.double().requires_grad_()
    ref = kda_layer_ref(p64, cfg, x64, keep_graph=True)
    (ref * wout.double()).sum().backward()
    errs = {"x": rel(xd.grad, x64.grad), "out": rel(out, ref)}
    for n, prm in m.named_parameters():
        errs[n] = rel(prm.grad, p64[n].grad)
    worst = max(errs, key=errs.get)
    print(f"layer training {dtype} T={T} d={hd}: out {errs['out']:.2e}, x grad {errs['x']:.2e}, "
          f"worst {worst} {errs[worst]:.2e}", flush=True)
    assert errs[worst] <= TOL_L[dtype], errs


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_layer_training_long_sequence(kda_pkg, dtype):
    """One sequence of 2048 tokens (64 checkpoint chunks carried backwards by the
    core's state kernel, 32 pre-processing tiles): every parameter's gradient
    and x's against autograd of the fp64 oracle."""
    m, cfg = _layer(kda_pkg, dtype, seed=13, head_dim=128, value_head_dim=128)
    B, T = 1, 2048
    print(f"layer training long sequence {dtype} B={B} T={T}", flush=True)
    gen = torch.Generator().manual_seed(14)
    x = torch.randn(B, T, 256, generator=gen).to(dtype)
    wout = torch.randn(B, T, 256, generator=gen)
    xd = x.to(DEV).requires_grad_()
    out = m(xd)
    (out.float() * wout.to(DEV)).sum().backward()
    p64 = {n: t.detach().double().cpu().requires_grad_() for n, t in m.state_dict().items()}
    x64 = x.double().requires_grad_()
    ref = kda_layer_ref(p64, cfg, x64, keep_graph=True)
    (ref * wout.double()).sum().backward()
    errs = {"x": rel(xd.grad, x64.grad), "out": rel(out, ref)}
    for n, prm in m.named_parameters():
        errs[n] = rel(prm.grad, p64[n].grad)
    worst = max(errs, key=errs.get)
    print(f"  out {errs['out']:.2e}, x grad {errs['x']:.2e}, worst {worst} {errs[worst]:.2e}", flush=True)
    assert errs[worst] <= TOL_L[dtype], errs


def test_layer_training_deterministic_and_rejects_cache(kda_pkg):
    """Two backward passes give bit-identical gradients (the token sums run in
    a fixed order); the training path takes no cache or state."""
    m, cfg = _layer(kda_pkg, torch.float16, seed=7)
    x = torch.randn(2, 96, 256, generator=torch.Generator().manual_seed(8)).to(torch.float16).to(DEV)
    grads = []
    for _ in range(2):
        m.zero_grad()
        m(x).float().square().mean().backward()
        grads.append({n: p.grad.clone() for n, p in m.named_parameters()})
    for n in grads[0]:
        assert torch.equal(grads[0][n], grads[1][n]), n
    with pytest.raises(kda_pkg.KdaError, match="cache"):
        m(x, use_cache=True)
