"""GPU parity of the gated core entry points (kda_chunkwise_gated, kda_recurrent_gated).

These fuse the KDA layer's gate pre-processing (``kimi_linear/kda.py:452-460``:
g = -exp(A_log) softplus(gk + dt_bias), beta = sigmoid(logit), in fp32) into
the kernels' loads.  The checker is the oracle's ``gates_ref`` (that formula,
pinned through the layer fixture written by the reference module) followed
by the core oracle: the same bars as the ungated parity tests (fp16 inputs:
o max-abs <= 2e-3, state relative error <= 1e-3; fp32: 1e-5).

The decay itself is checked in isolation: with beta = 0 and an all-ones
initial state, the final state of a call is the product of the per-token
decays, which must match exp(sum g) computed in fp64 to a few ulps per token,
over the whole range of z = gk + dt_bias (down to e^z far below fp32's
epsilon, up past torch's softplus threshold of 20) and A_log up to log 64.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import kda_chunkwise_ref, kda_recurrent_ref
from oracle.kda_layer_oracle import gates_ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
O_TOL = 2e-3
S_TOL = 1e-3


def max_abs(a, b):
    return (a.detach().double().cpu() - b.detach().double().cpu()).abs().max().item()


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm()).item()


def make(B, T, H, K, V, dtype, seed=0, a_log_range=(0.0, math.log(16.0)), state_std=None):
    """Layer-like core inputs with the gate given as gk and logits (activation
    dtype), A_log and dt_bias fp32 [H, K]; on the CPU."""
    gen = torch.Generator().manual_seed(seed)

    def randn(*shape):
        return torch.randn(*shape, generator=gen)

    q = F.normalize(randn(B, T, H, K), dim=-1).to(dtype)
    k = F.normalize(randn(B, T, H, K), dim=-1).to(dtype)
    v = randn(B, T, H, V).to(dtype)
    lo, hi = a_log_range
    a_log = torch.rand(H, K, generator=gen) * (hi - lo) + lo
    gk = randn(B, T, H, K).to(dtype)
    dt_bias = randn(H, K) * 0.1
    logit = randn(B, T, H).to(dtype)
    state = randn(B, H, K, V) * state_std if state_std is not None else None
    return dict(q=q, k=k, v=v, gk=gk, logit=logit, a_log=a_log, dt_bias=dt_bias, state=state)


def dev(inp):
    return {n: (t.to(DEV) if t is not None else None) for n, t in inp.items()}


def o_bar(dtype, o_ref):
    """O_TOL, plus one bf16 ulp of the largest output for bf16 (both outputs
    are rounded to bf16, 3 mantissa bits fewer than fp16)."""
    return O_TOL + (2.0 ** -7 * float(o_ref.float().abs().max()) if dtype == torch.bfloat16 else 0.0)


def oracle_gates(inp):
    return gates_ref(inp["gk"], inp["logit"], inp["a_log"], inp["dt_bias"])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,T,H,state", [(2, 256, 4, False), (1, 192, 2, True), (4, 128, 16, False),
                                         (1, 100, 2, True), (2, 10, 3, True)])
def test_chunkwise_gated_matches_oracle(kda_pkg, dtype, B, T, H, state):
    """V = 128 in one round of workgroups: the 64-column (NC = 4) kernel.
    T = 100 and 10 end in a partial block, whose padded rows must leave the
    state alone (chunk_size = T there)."""
    K = V = 128
    C = 64 if T % 64 == 0 else T
    inp = make(B, T, H, K, V, dtype, seed=1, state_std=0.05 if state else None)
    d = dev(inp)
    with torch.no_grad():
        o, s = kda_pkg.kda_chunkwise_gated(d["q"], d["k"], d["v"], d["gk"], d["logit"], d["a_log"], d["dt_bias"],
                                           initial_state=d["state"], chunk_size=C, state_dtype=torch.float32)
    g, beta = oracle_gates(inp)
    o_ref, s_ref = kda_chunkwise_ref(inp["q"], inp["k"], inp["v"], g, beta, initial_state=inp["state"],
                                     chunk_size=C, state_dtype=torch.float32)
    eo, es = max_abs(o, o_ref), rel(s, s_ref)
    print(f"gated chunkwise {dtype} B={B} T={T} H={H}: o max-abs {eo:.2e} state rel {es:.2e}", flush=True)
    assert eo <= o_bar(dtype, o_ref) and es <= S_TOL, (eo, es)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K,V,T", [(64, 96, 128), (128, 32, 100), (64, 16, 64)])
def test_chunkwise_gated_narrow_tiles_match_oracle(kda_pkg, dtype, K, V, T):
    """V not a multiple of 64: 32-column (NC = 2: V = 96, 32) and 16-column
    (NC = 1: V = 16) workgroups, whose producer waves also take the inverse
    of (I + L); T = 100 ends in a partial block."""
    B, H = 2, 4
    C = 64 if T % 64 == 0 else T
    inp = make(B, T, H, K, V, dtype, seed=7 + V, state_std=0.05)
    d = dev(inp)
    with torch.no_grad():
        o, s = kda_pkg.kda_chunkwise_gated(d["q"], d["k"], d["v"], d["gk"], d["logit"], d["a_log"], d["dt_bias"],
                                           initial_state=d["state"], chunk_size=C, state_dtype=torch.float32)
    g, beta = oracle_gates(inp)
    o_ref, s_ref = kda_chunkwise_ref(inp["q"], inp["k"], inp["v"], g, beta, initial_state=inp["state"],
                                     chunk_size=C, state_dtype=torch.float32)
    eo, es = max_abs(o, o_ref), rel(s, s_ref)
    print(f"gated chunkwise narrow tiles {dtype} K={K} V={V} T={T}: o max-abs {eo:.2e} state rel {es:.2e}",
          flush=True)
    assert eo <= o_bar(dtype, o_ref) and es <= S_TOL, (eo, es)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,T", [(8, 128), (16, 128), (8, 100), (16, 100)])
def test_chunkwise_gated_wide_launches_match_oracle(kda_pkg, dtype, B, T):
    """The gated tiles the layer's prefill runs at B=5-16 with 16 heads of 128:
    128 chains -> 64-column workgroups of four 16-column consumer waves
    (NC = 4); 256 chains -> 128-column workgroups whose consumer waves own two
    column groups (NC = 4, CG = 2, the plain output path).  T = 100 ends in a
    partial block (the layer's tail-free body is a multiple of 64; a direct
    call need not be).  Three (batch, head) pairs against the oracle, and
    every sequence's state against the same sequence run alone (16 chains,
    16-column workgroups: the same per-column arithmetic)."""
    H, K, V = 16, 128, 128
    C = 64 if T % 64 == 0 else T
    print(f"gated chunkwise wide launch {dtype} B={B} T={T} H={H}", flush=True)
    inp = make(B, T, H, K, V, dtype, seed=B + T, state_std=0.05)
    d = dev(inp)
    with torch.no_grad():
        o, s = kda_pkg.kda_chunkwise_gated(d["q"], d["k"], d["v"], d["gk"], d["logit"], d["a_log"], d["dt_bias"],
                                           initial_state=d["state"], chunk_size=C, state_dtype=torch.float32)
        one = {n: (t[B - 1:B] if t is not None and t.dim() >= 3 else t) for n, t in d.items()}
        o1, s1 = kda_pkg.kda_chunkwise_gated(one["q"], one["k"], one["v"], one["gk"], one["logit"], one["a_log"],
                                             one["dt_bias"], initial_state=one["state"], chunk_size=C,
                                             state_dtype=torch.float32)
    assert torch.equal(o[B - 1:B], o1) and torch.equal(s[B - 1:B], s1)
    g, beta = oracle_gates(inp)
    for b, h in ((0, 0), (B // 2, 7), (B - 1, 15)):
        sl = lambda t: t[b:b + 1, :, h:h + 1]  # noqa: E731
        o_ref, s_ref = kda_chunkwise_ref(sl(inp["q"]), sl(inp["k"]), sl(inp["v"]), sl(g),
                                         beta[b:b + 1, :, h:h + 1], initial_state=inp["state"][b:b + 1, h:h + 1],
                                         chunk_size=C, state_dtype=torch.float32)
        eo, es = max_abs(o[b:b + 1, :, h:h + 1], o_ref), rel(s[b:b + 1, h:h + 1], s_ref)
        print(f"  b={b} h={h}: o max-abs {eo:.2e} state rel {es:.2e}", flush=True)
        assert eo <= o_bar(dtype, o_ref) and es <= S_TOL, (b, h, eo, es)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_chunkwise_gated_equals_ungated_with_the_same_gates(kda_pkg, dtype):
    """The gated kernel and the ungated one fed g, beta from the oracle's formula
    (computed on the host) differ only by the decay's rounding."""
    B, T, H, K, V = 2, 320, 4, 64, 64
    inp = make(B, T, H, K, V, dtype, seed=2, state_std=0.02)
    d = dev(inp)
    g, beta = oracle_gates(inp)
    with torch.no_grad():
        o1, s1 = kda_pkg.kda_chunkwise_gated(d["q"], d["k"], d["v"], d["gk"], d["logit"], d["a_log"],
                                             d["dt_bias"], initial_state=d["state"], chunk_size=32,
                                             state_dtype=torch.float32)
        o2, s2 = kda_pkg.kda_chunkwise(d["q"], d["k"], d["v"], g.to(DEV), beta.to(DEV), initial_state=d["state"],
                                       chunk_size=32, state_dtype=torch.float32)
    eo, es = rel(o1, o2), rel(s1, s2)
    print(f"gated vs ungated {dtype}: o rel {eo:.2e} state rel {es:.2e}", flush=True)
    assert eo <= 1e-4 and es <= 1e-4, (eo, es)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_recurrent_gated_matches_oracle(kda_pkg, dtype):
    B, T, H, K, V = 3, 40, 4, 128, 128
    inp = make(B, T, H, K, V, dtype, seed=3, state_std=0.02)
    d = dev(inp)
    with torch.no_grad():
        o, s = kda_pkg.kda_recurrent_gated(d["q"], d["k"], d["v"], d["gk"], d["logit"], d["a_log"], d["dt_bias"],
                                           state=d["state"], state_dtype=torch.float32)
    g, beta = oracle_gates(inp)
    o_ref, s_ref = kda_recurrent_ref(inp["q"], inp["k"], inp["v"], g, beta, state=inp["state"],
                                     state_dtype=torch.float32)
    eo, es = rel(o, o_ref), rel(s, s_ref)
    print(f"gated recurrent {dtype}: o rel {eo:.2e} state rel {es:.2e}", flush=True)
    tol = 1e-5 if dtype == torch.float32 else 2e-3
    assert eo <= tol and es <= tol, (eo, es)


def test_chunkwise_gated_fp32_runs_the_recurrence(kda_pkg):
    """fp32 activations: the gated call is fp32 throughout (the gated recurrence)."""
    B, T, H, K, V = 1, 128, 2, 64, 64
    inp = make(B, T, H, K, V, torch.float32, seed=4, state_std=0.1)
    d = dev(inp)
    with torch.no_grad():
        o, s = kda_pkg.kda_chunkwise_gated(d["q"], d["k"], d["v"], d["gk"], d["logit"], d["a_log"], d["dt_bias"],
                                           initial_state=d["state"], chunk_size=64, state_dtype=torch.float32)
    g, beta = oracle_gates(inp)
    o_ref, s_ref = kda_chunkwise_ref(inp["q"], inp["k"], inp["v"], g, beta, initial_state=inp["state"],
                                     chunk_size=64, state_dtype=torch.float32)
    assert rel(o, o_ref) <= 1e-5 and rel(s, s_ref) <= 1e-5


def _decay_case(T, H, K, dtype, seed):
    """gk whose z = gk + dt_bias sits, per channel, near a level spread from -60
    to 40 over the channels; A_log from log 1 to log 64; logits that make beta
    exactly 0."""
    gen = torch.Generator().manual_seed(seed)
    a_log = torch.rand(H, K, generator=gen) * math.log(64.0)
    dt_bias = torch.randn(H, K, generator=gen) * 0.1
    level = torch.linspace(-60.0, 40.0, H * K)[torch.randperm(H * K, generator=gen)].reshape(H, K)
    z = level + 0.5 * torch.randn(1, T, H, K, generator=gen)
    gk = (z - dt_bias).to(dtype)
    logit = torch.full((1, T, H), -6.0e4).to(dtype)      # sigmoid -> 0 in fp32
    q = F.normalize(torch.randn(1, T, H, K, generator=gen), dim=-1).to(dtype)
    k = F.normalize(torch.randn(1, T, H, K, generator=gen), dim=-1).to(dtype)
    v = torch.randn(1, T, H, K, generator=gen).to(dtype)
    # the decay each token applies, in fp64 from the values the kernel reads
    zz = gk.double() + dt_bias.double()
    sp = torch.where(zz > 20, zz, torch.log1p(torch.exp(torch.clamp(zz, max=20))))
    g64 = -torch.exp(a_log.double()) * sp
    return dict(q=q, k=k, v=v, gk=gk, logit=logit, a_log=a_log, dt_bias=dt_bias), g64


@pytest.mark.parametrize("path", ["recurrent_f32", "recurrent_f16", "chunkwise_f16"])
def test_gated_decay_over_the_whole_gate_range(kda_pkg, path):
    """beta = 0 and S_0 = 1: the final state row of channel c is prod_t a_t(c).
    Per token the decay must be right to a few ulps of its exponent, from
    e^z < 1e-26 (where log(1 + e^z) in fp32 would round to 0) past z = 20."""
    dtype = torch.float32 if path.endswith("f32") else torch.float16
    T, H, K = (1, 4, 128) if path.startswith("recurrent") else (32, 2, 64)
    inp, g64 = _decay_case(T, H, K, dtype, seed=5)
    d = dev(inp)
    s0 = torch.ones(1, H, K, K, device=DEV)
    fn = kda_pkg.kda_recurrent_gated if path.startswith("recurrent") else kda_pkg.kda_chunkwise_gated
    kw = dict(state=s0) if path.startswith("recurrent") else dict(initial_state=s0, chunk_size=T)
    with torch.no_grad():
        _, s = fn(d["q"], d["k"], d["v"], d["gk"], d["logit"], d["a_log"], d["dt_bias"],
                  state_dtype=torch.float32, **kw)
    got = s[0, :, :, 0].double().cpu()                    # [H, K]: every column is the same
    assert torch.equal(s[0].cpu(), s[0, :, :, :1].cpu().expand(H, K, K))
    logsum = g64[0].sum(0)                                # [H, K], log of the exact product
    want = torch.exp(logsum)
    live = logsum > -80.0                                 # products above fp32's normal range
    # per channel, a few ulps of the exponent per token: T (1 + |log prod|) 2^-21
    # (the form without the rounding correction of log2(1 + t) exceeds this
    # by 2.5-7x on these inputs, the corrected one stays below 0.4x on the CPU)
    err = (got - want).abs() / want
    ratio = (err / ((T * 2.0 ** -21) * (1.0 + logsum.abs())))[live].max().item()
    print(f"{path}: {int(live.sum())} live channels, max error / bound {ratio:.2f}", flush=True)
    assert ratio <= 1.0, ratio
    assert (got[~live] <= 1e-30).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K,V,T", [(128, 128, 192), (64, 64, 128), (128, 64, 100), (64, 128, 64),
                                   (128, 128, 96), (64, 128, 160)])   # odd chunk counts: a padded last chunk
def test_chunkwise_fused_matches_gated_plus_output_kernel(kda_pkg, dtype, K, V, T):
    """The output epilogue on the chunk kernel's tiles (one workgroup per head,
    4 consumer waves of V / 64 column groups) against the gated chunk kernel
    followed by the separate output kernel: the state bit for bit (same
    arithmetic per column), y within an output ulp or two (the row sums of
    squares are added in another order)."""
    import importlib
    ops = importlib.import_module("kimi_linear_amd.layer_ops")
    B, H = 2, 3
    inp = make(B, T, H, K, V, dtype, seed=9, state_std=0.05)
    d = dev(inp)
    gen = torch.Generator().manual_seed(10)
    og = torch.randn(B, T, H * V, generator=gen).to(dtype).to(DEV)
    w = (1 + 0.1 * torch.randn(H, V, generator=gen)).to(DEV)
    C = 64 if T % 64 == 0 else T
    with torch.no_grad():
        y, s1 = kda_pkg.kda_chunkwise_fused(d["q"], d["k"], d["v"], d["gk"], d["logit"], d["a_log"], d["dt_bias"],
                                            og, w, 1e-5, initial_state=d["state"], chunk_size=C,
                                            state_dtype=torch.float32)
        o, s2 = kda_pkg.kda_chunkwise_gated(d["q"], d["k"], d["v"], d["gk"], d["logit"], d["a_log"], d["dt_bias"],
                                            initial_state=d["state"], chunk_size=C, state_dtype=torch.float32)
        y_ref = ops.kda_output(o, og, w, 1e-5)
    assert torch.equal(s1, s2)
    err = ((y.double() - y_ref.double()).abs() / y_ref.double().abs().clamp(min=1.0)).max().item()
    tol = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}[dtype]
    print(f"fused epilogue {dtype} K={K} V={V} T={T}: y err {err:.2e}", flush=True)
    assert err <= tol, err
