"""GPU parity of the native chunkwise backward (kda_chunkwise and
kda_recurrent under autograd).

Reference: autograd of the oracle ``kda_chunkwise_ref`` in fp64 on the CPU
(pinned by finite differences and by the recurrence in
tests/test_oracle_backward.py).  The loss is <o, W_o> + <S_T, W_S> for fixed
random weights, so every gradient path -- through the outputs, the final
state and the initial state -- is exercised.

Tolerance: relative L2 error <= 1e-4 per gradient for fp32 inputs (their
checkpoints are fp32-exact: the fp32 token recurrence's states and an fp32
kernel's R, A, L, N; the backward's products are bf16 pairs, ~2^-17
relative; measured 4e-6 to 2.4e-5), 2e-3 for fp16 inputs and 1e-2 for bf16
inputs (the checkpoints come from the fp16-operand chunk pipeline and the
gradients are rounded to that dtype, 2^-11 and 2^-8 relative; measured
~3.2e-4 and ~2.3e-3).
"""

from __future__ import annotations

import pytest
import torch

from oracle import kda_chunkwise_ref, kda_recurrent_ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
NAMES = ("q", "k", "v", "g", "beta", "s0")


def _tol(dtype):
    return {torch.float32: 1e-4, torch.float16: 2e-3, torch.bfloat16: 1e-2}[dtype]


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


@pytest.fixture(scope="module")
def wl(kda_pkg):
    import importlib
    return importlib.import_module("kimi_linear_amd.workloads")


def _case(wl, B, T, H, K, V, seed, dtype, state):
    inp = wl.make_inputs(B, T, H, K, V, seed=seed, qkv_dtype=dtype,
                         state_std=0.02 if state else None)
    gen = torch.Generator().manual_seed(seed + 7)
    wo = torch.randn(B, T, H, V, generator=gen, dtype=torch.float64)
    ws = torch.randn(B, H, K, V, generator=gen, dtype=torch.float64)
    return [inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["state"]], wo, ws


def _ref_grads(xs, wo, ws, chunk):
    leaves = [x.double().clone().requires_grad_(True) if x is not None else None for x in xs]
    T = xs[0].shape[1]
    # the oracle needs T % chunk == 0 like the reference; any chunk dividing T gives the same function
    o, s = kda_chunkwise_ref(*leaves[:5], initial_state=leaves[5], chunk_size=chunk, state_dtype=torch.float64)
    ((o * wo).sum() + (s * ws).sum()).backward()
    assert T % chunk == 0
    return [x.grad if x is not None else None for x in leaves]


def _native_grads(pkg, xs, wo, ws, chunk):
    leaves = [x.to(DEV).clone().requires_grad_(True) if x is not None else None for x in xs]
    o, s = pkg.kda_chunkwise(*leaves[:5], initial_state=leaves[5], chunk_size=chunk,
                             state_dtype=torch.float32)
    ((o.float() * wo.to(DEV, torch.float32)).sum() + (s * ws.to(DEV, torch.float32)).sum()).backward()
    torch.cuda.synchronize()
    return [x.grad if x is not None else None for x in leaves]


@pytest.mark.parametrize("B,T,H,K,V,chunk,state", [
    (1, 64, 2, 32, 32, 32, False),
    (2, 80, 2, 64, 64, 16, True),      # 2.5 checkpoint chunks: a ragged last chunk
    (1, 128, 1, 128, 128, 64, True),
    (1, 16, 3, 128, 64, 16, True),     # a single partial chunk
])
def test_backward_fp32(kda_pkg, wl, B, T, H, K, V, chunk, state):
    print(f"backward fp32 B={B} T={T} H={H} K={K} V={V} chunk={chunk} state={state}", flush=True)
    xs, wo, ws = _case(wl, B, T, H, K, V, seed=100 + K + T, dtype=torch.float32, state=state)
    ref = _ref_grads(xs, wo, ws, chunk)
    got = _native_grads(kda_pkg, xs, wo, ws, chunk)
    for name, a, r in zip(NAMES, got, ref):
        if r is None:
            assert a is None
            continue
        assert a.dtype == xs[NAMES.index(name)].dtype and a.shape == r.shape
        err = _rel(a, r)
        print(f"  d{name}: rel {err:.2e}", flush=True)
        assert err <= 1e-4, (name, err)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_backward_half(kda_pkg, wl, dtype):
    """q, k, v, d_o and dq, dk, dv in the activation dtype, read and written as such."""
    B, T, H, K, V = 1, 96, 2, 64, 64
    print(f"backward {dtype} B={B} T={T} H={H} K={K} V={V}", flush=True)
    xs, wo, ws = _case(wl, B, T, H, K, V, seed=5, dtype=dtype, state=True)
    ref = _ref_grads(xs, wo, ws, 32)
    got = _native_grads(kda_pkg, xs, wo, ws, 32)
    for name, a, r in zip(NAMES, got, ref):
        err = _rel(a, r)
        print(f"  d{name}: rel {err:.2e}", flush=True)
        assert err <= _tol(dtype), (name, err)


def test_backward_state_only_loss(kda_pkg, wl):
    """Only the final state enters the loss: the output gradient is zero."""
    xs, _, ws = _case(wl, 1, 64, 2, 64, 64, seed=9, dtype=torch.float32, state=True)
    leaves = [x.double().clone().requires_grad_(True) for x in xs]
    _, s = kda_chunkwise_ref(*leaves[:5], initial_state=leaves[5], chunk_size=32, state_dtype=torch.float64)
    (s * ws).sum().backward()
    dev = [x.to(DEV).clone().requires_grad_(True) for x in xs]
    _, s2 = kda_pkg.kda_chunkwise(*dev[:5], initial_state=dev[5], chunk_size=32, state_dtype=torch.float32)
    (s2 * ws.to(DEV, torch.float32)).sum().backward()
    for name, a, r in zip(NAMES, dev, leaves):
        if r.grad is None:
            # q only reaches the outputs: its gradient is zero
            assert a.grad is None or not a.grad.any(), name
            continue
        err = _rel(a.grad, r.grad)
        assert err <= 1e-4, (name, err)


def test_backward_matches_eager_chaining(kda_pkg, wl):
    """Gradients through two chained calls (state handed over) equal one call's."""
    xs, wo, ws = _case(wl, 1, 128, 2, 64, 64, seed=21, dtype=torch.float32, state=True)
    one = _native_grads(kda_pkg, xs, wo, ws, 32)
    leaves = [x.to(DEV).clone().requires_grad_(True) for x in xs]
    q, k, v, g, beta, s0 = leaves
    o1, s1 = kda_pkg.kda_chunkwise(q[:, :64], k[:, :64], v[:, :64], g[:, :64], beta[:, :64],
                                   initial_state=s0, chunk_size=32, state_dtype=torch.float32)
    o2, s2 = kda_pkg.kda_chunkwise(q[:, 64:], k[:, 64:], v[:, 64:], g[:, 64:], beta[:, 64:],
                                   initial_state=s1, chunk_size=32, state_dtype=torch.float32)
    o = torch.cat([o1, o2], dim=1)
    ((o * wo.to(DEV, torch.float32)).sum() + (s2 * ws.to(DEV, torch.float32)).sum()).backward()
    for name, a, b in zip(NAMES, [x.grad for x in leaves], one):
        err = _rel(a, b)
        assert err <= 1e-4, (name, err)


@pytest.mark.parametrize("H,K,V,dtype", [(2, 64, 64, torch.float32), (2, 64, 64, torch.float16),
                                         (1, 128, 128, torch.float16)])
def test_backward_long_sequence(kda_pkg, wl, H, K, V, dtype):
    """T = 2048: the state kernel carries dS backwards over 64 checkpoint
    chunks (with the next chunk fetched while the current one is computed),
    as in the training workload.  Against the fp64 oracle's autograd (chunk
    16), and one T = 2048 call against two chained T = 1024 calls."""
    B, T = 1, 2048
    print(f"backward long sequence {dtype} B={B} T={T} H={H} K={K} V={V}", flush=True)
    xs, wo, ws = _case(wl, B, T, H, K, V, seed=300 + K, dtype=dtype, state=True)
    ref = _ref_grads(xs, wo, ws, 16)
    got = _native_grads(kda_pkg, xs, wo, ws, 64)
    tol = _tol(dtype)
    for name, a, r in zip(NAMES, got, ref):
        err = _rel(a, r)
        print(f"  d{name}: rel {err:.2e}", flush=True)
        assert err <= tol, (name, err)
    leaves = [x.to(DEV).clone().requires_grad_(True) for x in xs]
    q, k, v, g, beta, s0 = leaves
    h = T // 2
    o1, s1 = kda_pkg.kda_chunkwise(q[:, :h], k[:, :h], v[:, :h], g[:, :h], beta[:, :h],
                                   initial_state=s0, chunk_size=64, state_dtype=torch.float32)
    o2, s2 = kda_pkg.kda_chunkwise(q[:, h:], k[:, h:], v[:, h:], g[:, h:], beta[:, h:],
                                   initial_state=s1, chunk_size=64, state_dtype=torch.float32)
    o = torch.cat([o1, o2], dim=1)
    ((o.float() * wo.to(DEV, torch.float32)).sum() + (s2 * ws.to(DEV, torch.float32)).sum()).backward()
    for name, a, b in zip(NAMES, [x.grad for x in leaves], got):
        err = _rel(a, b)
        print(f"  chained vs one call d{name}: rel {err:.2e}", flush=True)
        # the two halves' checkpoints and gradients are computed as in one call
        # (the state enters the second half as fp32), up to output rounding
        assert err <= (1e-4 if dtype == torch.float32 else 2e-3), (name, err)


def test_backward_unsupported_head_dims_raise(kda_pkg, wl):
    inp = wl.make_inputs(1, 16, 1, 16, 32, seed=3)
    q = inp["q"].to(DEV).requires_grad_(True)
    with pytest.raises(kda_pkg.KdaError, match="backward supports"):
        kda_pkg.kda_chunkwise(q, inp["k"].to(DEV), inp["v"].to(DEV), inp["g"].to(DEV), inp["beta"].to(DEV),
                              chunk_size=16)


# (6, 128, 128): 96 chains, where 32-column state workgroups would need a
# second round, so the state kernel runs 64-column ones (and the forward one
# round of 64-column workgroups)
@pytest.mark.parametrize("B,K,V,dtype", [(16, 64, 64, torch.float32), (9, 64, 128, torch.float16),
                                         (9, 128, 128, torch.float16), (6, 128, 128, torch.float16)])
def test_backward_wide_launch_matches_per_sequence(kda_pkg, wl, B, K, V, dtype):
    """256 (batch, head) chains of 64 columns: the checkpointing forward runs its
    widest instantiation (four 16-column consumer waves a workgroup; at V=128
    and 144 chains, 128-column workgroups of two column groups a wave) and the
    gradients come from its checkpoints; the state kernel runs 64-column
    workgroups (at K = V = 128 fp16: the instantiations of the B=8 T=4096 H=16
    training workload).  They must equal the gradients of the same sequences
    run one at a time (16 chains: one-wave forward, 32-column state kernel),
    and sequence 0 must match the fp64 oracle."""
    T, H = 64, 16
    print(f"backward wide launch B={B} T={T} H={H} K={K} V={V} {dtype}", flush=True)
    xs, wo, ws = _case(wl, B, T, H, K, V, seed=31, dtype=dtype, state=True)
    wide = _native_grads(kda_pkg, xs, wo, ws, 32)
    for b in (0, 7, B - 1):
        sub = [x[b:b + 1] for x in xs]
        one = _native_grads(kda_pkg, sub, wo[b:b + 1], ws[b:b + 1], 32)
        for name, a, r in zip(NAMES, wide, one):
            err = _rel(a[b:b + 1], r)
            assert err <= 1e-6, (b, name, err)
    ref = _ref_grads([x[:1] for x in xs], wo[:1], ws[:1], 32)
    tol = _tol(dtype)
    for name, a, r in zip(NAMES, wide, ref):
        err = _rel(a[:1], r)
        print(f"  d{name}: rel {err:.2e}", flush=True)
        assert err <= tol, (name, err)


def _native_rec_grads(pkg, xs, wo, ws):
    leaves = [x.to(DEV).clone().requires_grad_(True) if x is not None else None for x in xs]
    o, s = pkg.kda_recurrent(*leaves[:5], state=leaves[5], state_dtype=torch.float32)
    ((o.double() * wo.to(DEV)).sum() + (s.double() * ws.to(DEV)).sum()).backward()
    torch.cuda.synchronize()
    return [x.grad if x is not None else None for x in leaves]


def _ref_rec_grads(xs, wo, ws, dtype=torch.float64):
    leaves = [(x.to(dtype) if dtype is not None else x).clone().requires_grad_(True) if x is not None else None
              for x in xs]
    o, s = kda_recurrent_ref(*leaves[:5], state=leaves[5], state_dtype=torch.float64)
    ((o.double() * wo).sum() + (s.double() * ws).sum()).backward()
    return [x.grad if x is not None else None for x in leaves]


@pytest.mark.parametrize("B,T,H,K,V,dtype,state", [
    (1, 37, 2, 64, 64, torch.float32, True),      # T a multiple of no chunk size
    (2, 5, 3, 128, 32, torch.float32, False),
    (3, 1, 4, 32, 64, torch.float32, True),       # one decode step
    (1, 50, 2, 64, 64, torch.bfloat16, True),
])
def test_recurrent_backward(kda_pkg, wl, B, T, H, K, V, dtype, state):
    """kda_recurrent under autograd (kda.py:188-219 is differentiated by torch's
    autograd in the reference) against autograd of the fp64 recurrence oracle;
    gradients keep the inputs' dtypes."""
    print(f"recurrent backward B={B} T={T} H={H} K={K} V={V} {dtype} state={state}", flush=True)
    xs, wo, ws = _case(wl, B, T, H, K, V, seed=200 + T, dtype=dtype, state=state)
    ref = _ref_rec_grads(xs, wo, ws)
    got = _native_rec_grads(kda_pkg, xs, wo, ws)
    tol = _tol(dtype)
    for name, x, a, r in zip(NAMES, xs, got, ref):
        if r is None:
            assert a is None
            continue
        assert a.dtype == x.dtype and a.shape == r.shape
        err = _rel(a, r)
        print(f"  d{name}: rel {err:.2e}", flush=True)
        assert err <= tol, (name, err)


def test_recurrent_backward_fp16_clamp(kda_pkg, wl):
    """An fp16 o is clamped to +-60000 (kda.py:217-218) and a clamped entry
    passes no gradient.  With beta = 1 and unit keys, k_t^T S_t = v_t, so
    q = 32 k (q~ = 4 k) gives o_t = 4 v_t exactly: v[..., 0] = 25000 puts
    column 0 of o at 1e5, far past the clamp, the other columns at 4 v.  The
    final-state weight of column 0 is zero, so every gradient of column 0
    comes through the clamped outputs: an unmasked d_o would show in dv[..., 0]
    (4 w_o instead of 0) and in dq, dk, dg."""
    B, T, H, K, V = 1, 12, 2, 64, 32
    inp = wl.make_inputs(B, T, H, K, V, seed=41, qkv_dtype=torch.float16)
    k = inp["k"]
    q = (k.float() * 32).half()
    v = inp["v"].clone()
    v[..., 0] = 25000.0
    beta = torch.ones(B, T, H)
    xs = [q, k, v, inp["g"], beta, None]
    gen = torch.Generator().manual_seed(43)
    wo = torch.randn(B, T, H, V, generator=gen, dtype=torch.float64)
    ws = torch.randn(B, H, K, V, generator=gen, dtype=torch.float64)
    ws[..., 0] = 0.0
    with torch.no_grad():
        o, _ = kda_pkg.kda_recurrent(*[x.to(DEV) for x in xs[:5]], state_dtype=torch.float32)
    assert bool((o[..., 0].float() == 60000.0).all()) and float(o[..., 1:].float().abs().max()) < 100
    ref = _ref_rec_grads(xs, wo, ws, dtype=None)
    got = _native_rec_grads(kda_pkg, xs, wo, ws)
    assert float(got[2][..., 0].abs().max()) == 0.0
    for name, a, r in zip(NAMES[:5], got, ref):
        err = _rel(a, r)
        print(f"  d{name}: rel {err:.2e}", flush=True)
        assert err <= _tol(torch.float16), (name, err)


def test_fp16_record_holds_the_state_in_fp16_tiles(kda_pkg, wl):
    """fp16 activations: each chunk record's state is fp16 in 16 x 16 tiles in
    accumulator order in the first half of its K x V fp32 rows (element
    (r, c) at half ((r//16)(V//16) + c//16) 256 + (r%4) 64 + ((r//4)%4) 16 +
    c%16), as the header documents.  Chunk 0's record holds the initial state
    as given, rounded to fp16; R's rows follow the state's fp32 rows."""
    import importlib
    kda = importlib.import_module("kimi_linear_amd.kda")
    B, T, H, K, V = 1, 64, 2, 64, 96
    inp = wl.make_inputs(B, T, H, K, V, seed=61, qkv_dtype=torch.float16, state_std=0.5)
    d = {n: (x.to(DEV) if x is not None else None) for n, x in inp.items()}
    with torch.no_grad():
        _, _, ck = kda._forward("chunkwise", d["q"], d["k"], d["v"], d["g"], d["beta"], d["state"], 64,
                                torch.float32, ckpt=True)
    assert ck.shape == (B, H, 2, kda.ckpt_record(K, V))
    halves = ck[..., : K * V // 2].contiguous().view(torch.float16).cpu()     # [B, H, 2, K * V]
    r = torch.arange(K)[:, None]
    c = torch.arange(V)[None, :]
    off = ((r // 16) * (V // 16) + c // 16) * 256 + (r % 4) * 64 + ((r // 4) % 4) * 16 + c % 16
    s0 = halves[:, :, 0][..., off]                                             # [B, H, K, V]
    assert torch.equal(s0, inp["state"].half())


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_backward_completes_n_in_the_records(kda_pkg, wl, dtype):
    """The forward's records hold N's diagonal blocks (and zeros above them);
    kda_chunkwise_bwd completes the block below them in place.  After a
    backward every record's N is (I + Diag(beta) L)^-1 of that record's L,
    with beta = 0 past T (a ragged last chunk here), and a second backward
    over the same record returns the same gradients."""
    import importlib
    kda = importlib.import_module("kimi_linear_amd.kda")
    B, T, H, K, V = 2, 100, 3, 64, 64
    inp = wl.make_inputs(B, T, H, K, V, seed=71, qkv_dtype=dtype, state_std=0.1)
    d = {n: (x.to(DEV) if x is not None else None) for n, x in inp.items()}
    with torch.no_grad():
        _, _, ck = kda._forward("chunkwise", d["q"], d["k"], d["v"], d["g"], d["beta"], d["state"], 4,
                                torch.float32, ckpt=True)
        d_o = torch.randn(B, T, H, V, generator=torch.Generator().manual_seed(72)).to(dtype).to(DEV)
        g1 = kda._chunkwise_backward(d["q"], d["k"], d["v"], d["g"], d["beta"], ck, d_o, None, True)
        g2 = kda._chunkwise_backward(d["q"], d["k"], d["v"], d["g"], d["beta"], ck, d_o, None, True)
    torch.cuda.synchronize()
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)
    nck = -(-T // 32)
    mats = ck[..., (K + 32) * V:].reshape(B, H, nck, 3, 32, 32).double().cpu()
    L, N = mats[:, :, :, 1].tril(-1), mats[:, :, :, 2]
    beta = torch.zeros(B, H, nck * 32, dtype=torch.float64)
    beta[:, :, :T] = inp["beta"].double().permute(0, 2, 1)
    beta = beta.view(B, H, nck, 32)
    eye = torch.eye(32, dtype=torch.float64)
    resid = (N @ (eye + beta[..., :, None] * L) - eye).abs().max().item()
    print(f"record N {dtype}: max |N (I + Diag(beta) L) - I| {resid:.2e}", flush=True)
    assert resid < 1e-4, resid
