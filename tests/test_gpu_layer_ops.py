"""GPU parity of the fused layer kernels (kda_prep_fwd, kda_output_fwd) against
the layer oracle's pieces on the same inputs.

Each output is rounded once from fp32, so the bound is a few units in the last
place of the output dtype: max |err| <= tol * max(1, |ref|) with tol 5e-6
(fp32), 2e-3 (fp16), 1.6e-2 (bf16).  g and beta are fp32 for every input
dtype: 1e-5 (exp and log1p of the hardware exponential vs the CPU's).
"""

from __future__ import annotations

import pytest
import torch

from oracle.kda_layer_oracle import head_rmsnorm_ref, l2norm_ref, short_conv_ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL = {torch.float32: 5e-6, torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


@pytest.fixture(scope="module")
def ops(kda_pkg):
    import importlib
    return importlib.import_module("kimi_linear_amd.layer_ops")


def close(got, ref, tol):
    got, ref = got.detach().double().cpu(), ref.detach().double().cpu()
    err = ((got - ref).abs() / ref.abs().clamp(min=1.0)).max().item() if ref.numel() else 0.0
    return err <= tol, err


def prep_ref(xs, ws, bs, gk, a_log, dt_bias, beta_logit, H, K, V, eps, hist=None):
    """fp32 CPU result from the same (rounded) inputs."""
    B, T = xs[0].shape[:2]
    outs = []
    for i, (x, w, b) in enumerate(zip(xs, ws, bs)):
        h = hist[i].float().cpu() if hist is not None else None
        u = short_conv_ref(x.float().cpu(), w.float().cpu(), None if b is None else b.float().cpu(), history=h)
        s = u * torch.sigmoid(u)
        Dh = V if i == 2 else K
        s = s.view(B, T, H, Dh)
        outs.append(l2norm_ref(s, eps) if i < 2 else s)
    z = gk.float().cpu() + dt_bias.float().cpu().reshape(-1)
    sp = torch.where(z > 20, z, torch.log1p(torch.exp(torch.clamp(z, max=20))))
    g = (-torch.exp(a_log.float().cpu().reshape(-1)) * sp).view(B, T, H, K)
    beta = torch.sigmoid(beta_logit.float().cpu())
    return outs + [g, beta]


def make_prep_inputs(B, T, H, K, V, cs, dtype, seed, bias=True, strided=False):
    gen = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    Dk, Dv = H * K, H * V
    if strided:
        # views into one fused projection output [B, T, 2Dk + Dv + Dk + H]
        big = rn(B, T, 3 * Dk + Dv + H).to(dtype).to(DEV)
        q_in, k_in, v_in = big[..., :Dk], big[..., Dk:2 * Dk], big[..., 2 * Dk:2 * Dk + Dv]
        gk, beta_logit = big[..., 2 * Dk + Dv:3 * Dk + Dv], big[..., 3 * Dk + Dv:]
    else:
        q_in, k_in, v_in = (rn(B, T, D).to(dtype).to(DEV) for D in (Dk, Dk, Dv))
        gk, beta_logit = rn(B, T, Dk).to(dtype).to(DEV), (rn(B, T, H) * 2).to(dtype).to(DEV)
    ws = [(rn(D, 1, cs) * 0.5).to(dtype).to(DEV) for D in (Dk, Dk, Dv)]
    bs = [(rn(D) * 0.1).to(dtype).to(DEV) if bias else None for D in (Dk, Dk, Dv)]
    a_log = (torch.rand(H, K, generator=gen) * 2.77).to(DEV)
    dt_bias = (rn(H, K) * 0.1).to(DEV)
    return (q_in, k_in, v_in), ws, bs, gk, a_log, dt_bias, beta_logit


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 37, 2, 128, 128, 4), (1, 16, 3, 64, 128, 4), (3, 5, 1, 256, 64, 2),
                                   (2, 1, 2, 128, 128, 4), (1, 33, 2, 128, 128, 1)])
def test_prep_vs_oracle(ops, dtype, shape):
    B, T, H, K, V, cs = shape
    xs, ws, bs, gk, a_log, dt_bias, beta_logit = make_prep_inputs(B, T, H, K, V, cs, dtype, seed=T + K)
    with torch.no_grad():
        got = ops.kda_prep(*xs, ws, bs, gk, a_log, dt_bias, beta_logit, num_heads=H, head_dim=K,
                           value_head_dim=V, l2_eps=1e-6)
    ref = prep_ref(xs, ws, bs, gk, a_log, dt_bias, beta_logit, H, K, V, 1e-6)
    for name, gt, rf in zip(("q", "k", "v", "g", "beta"), got[:5], ref):
        tol = TOL[dtype] if name in "qkv" else 1e-5
        ok, err = close(gt, rf, tol)
        print(f"[prep {dtype} {shape} {name}] err {err:.2e}", flush=True)
        assert ok, (name, err)
    assert got[0].dtype == dtype and got[3].dtype == torch.float32 and got[5] is None


@pytest.mark.parametrize("T", [1, 7, 16, 40])
def test_prep_conv_cache(ops, T):
    """History in, new cache out (fresh tensors; in place for T <= 16), strided
    projection views; equal to convolving the concatenated sequence."""
    B, H, K, V, cs = 2, 2, 128, 128, 4
    dtype = torch.float16
    xs, ws, bs, gk, a_log, dt_bias, beta_logit = make_prep_inputs(B, T, H, K, V, cs, dtype, seed=50 + T,
                                                                  strided=True)
    gen = torch.Generator().manual_seed(60 + T)
    hist = [torch.randn(B, cs - 1, D, generator=gen).to(dtype).to(DEV) for D in (H * K, H * K, H * V)]
    hd = dict(zip("qkv", hist))
    with torch.no_grad():
        got = ops.kda_prep(*xs, ws, bs, gk, a_log, dt_bias, beta_logit, num_heads=H, head_dim=K,
                           value_head_dim=V, l2_eps=1e-6, hist=hd, want_hist=True)
    ref = prep_ref(xs, ws, bs, gk, a_log, dt_bias, beta_logit, H, K, V, 1e-6, hist=hist)
    for name, gt, rf in zip("qkv", got[:3], ref[:3]):
        ok, err = close(gt, rf, TOL[dtype])
        assert ok, (name, err)
    for i, n in enumerate("qkv"):
        full = torch.cat([hist[i], xs[i]], 1)
        assert torch.equal(got[5][n], full[:, -(cs - 1):])
    if T <= 16:
        inplace = {n: t.clone() for n, t in hd.items()}
        with torch.no_grad():
            got2 = ops.kda_prep(*xs, ws, bs, gk, a_log, dt_bias, beta_logit, num_heads=H, head_dim=K,
                                value_head_dim=V, l2_eps=1e-6, hist=inplace, hist_out=inplace)
        for a, b in zip(got[:5], got2[:5]):
            assert torch.equal(a, b)
        for n in "qkv":
            assert torch.equal(inplace[n], got[5][n])
    else:
        with torch.no_grad(), pytest.raises(Exception, match="overlap"):
            ops.kda_prep(*xs, ws, bs, gk, a_log, dt_bias, beta_logit, num_heads=H, head_dim=K,
                         value_head_dim=V, l2_eps=1e-6, hist=hd, hist_out=hd)


def test_prep_zero_rows_stay_finite(ops):
    """An all-zero q/k head (no bias) hits the eps clamp: 0 * 1/eps = 0."""
    B, T, H, K, V, cs = 1, 4, 1, 128, 128, 4
    xs, ws, bs, gk, a_log, dt_bias, beta_logit = make_prep_inputs(B, T, H, K, V, cs, torch.float32, seed=3,
                                                                  bias=False)
    xs = (torch.zeros_like(xs[0]), xs[1], xs[2])
    with torch.no_grad():
        q = ops.kda_prep(*xs, ws, bs, gk, a_log, dt_bias, beta_logit, num_heads=H, head_dim=K,
                         value_head_dim=V, l2_eps=1e-6)[0]
    assert torch.equal(q, torch.zeros_like(q))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("V", [64, 128, 256])
def test_output_vs_oracle(ops, dtype, V):
    B, T, H = 2, 9, 3
    gen = torch.Generator().manual_seed(V)
    o = (torch.randn(B, T, H, V, generator=gen) * 0.05).to(dtype)
    gate = torch.randn(B, T, H * V, generator=gen).to(dtype)
    w = (1 + 0.1 * torch.randn(H, V, generator=gen)).to(dtype)
    with torch.no_grad():
        y = ops.kda_output(o.to(DEV), gate.to(DEV), w.to(DEV), 1e-6)
    n = head_rmsnorm_ref(o.float(), w.float(), 1e-6).to(dtype).float()    # HeadwiseRMSNorm rounds to o's dtype
    ref = (n * torch.sigmoid(gate.float().view(B, T, H, V))).reshape(B, T, H * V)
    ok, err = close(y, ref, TOL[dtype])
    print(f"[output {dtype} V={V}] err {err:.2e}", flush=True)
    assert ok and y.dtype == dtype


def test_output_strided_core_view(ops):
    """o may be a strided view (the body slice of a longer output)."""
    gen = torch.Generator().manual_seed(5)
    full = torch.randn(2, 40, 2, 128, generator=gen).half().to(DEV)
    gate = torch.randn(2, 32, 256, generator=gen).half().to(DEV)
    w = torch.ones(2, 128, device=DEV, dtype=torch.float16)
    with torch.no_grad():
        y1 = ops.kda_output(full[:, :32], gate, w, 1e-6)
        y2 = ops.kda_output(full[:, :32].contiguous(), gate, w, 1e-6)
    assert torch.equal(y1, y2)


def test_prep_gate_softplus_tails(ops):
    """The forget gate over the whole softplus range: for z = gk + dt_bias far
    below 0, softplus(z) ~ e^z (not 0), and above the threshold 20 it is z
    (torch's rule).  Relative error per element <= 1e-5 against log1p(exp(z))."""
    B, T, H, K, V, cs = 1, 16, 2, 128, 128, 4
    xs, ws, bs, _, a_log, dt_bias, beta_logit = make_prep_inputs(B, T, H, K, V, cs, torch.float32, seed=77)
    z = torch.linspace(-60.0, 40.0, B * T * H * K, dtype=torch.float64).view(B, T, H * K)
    gk = (z - dt_bias.double().cpu().reshape(-1)).float().to(DEV)
    with torch.no_grad():
        got = ops.kda_prep(*xs, ws, bs, gk, a_log, dt_bias, beta_logit, num_heads=H, head_dim=K,
                           value_head_dim=V, l2_eps=1e-6)
    zf = gk.double().cpu() + dt_bias.double().cpu().reshape(-1)
    sp = torch.where(zf > 20, zf, torch.log1p(torch.exp(torch.clamp(zf, max=20))))
    ref = (-torch.exp(a_log.double().cpu().reshape(-1)) * sp).view(B, T, H, K)
    err = ((got[3].double().cpu() - ref).abs() / ref.abs()).max().item()
    print(f"[prep softplus tails] max rel err {err:.2e}", flush=True)
    assert (got[3] < 0).all() and err <= 1e-5


@pytest.mark.parametrize("T", [1, 37])
def test_prep_without_gates_matches_prep_with_gates(ops, T):
    """A call that leaves the gates to the core (gk=None) writes the same q, k, v
    and conv cache, bit for bit, and returns no g and beta."""
    B, H, K, V, cs = 2, 2, 128, 128, 4
    xs, ws, bs, gk, a_log, dt_bias, beta_logit = make_prep_inputs(B, T, H, K, V, cs, torch.float16, seed=11)
    kw = dict(num_heads=H, head_dim=K, value_head_dim=V, l2_eps=1e-6, want_hist=True)
    q1, k1, v1, g1, b1, h1 = ops.kda_prep(*xs, ws, bs, gk, a_log, dt_bias, beta_logit, **kw)
    q2, k2, v2, g2, b2, h2 = ops.kda_prep(*xs, ws, bs, None, None, None, None, **kw)
    assert g2 is None and b2 is None and g1 is not None
    for a, b in ((q1, q2), (k1, k2), (v1, v2)) + tuple((h1[n], h2[n]) for n in "qkv"):
        assert torch.equal(a, b)
