"""GPU parity of the HIP KDA kernels against the CPU oracle.

Tolerances (fp16 inputs, fp32 accumulation and state): output max-abs <= 2e-3,
final-state relative error <= 1e-3.  The all-fp32 recurrence is held to 1e-5.
bf16 inputs: the same state bar, and the output bar plus one bf16 ulp of the
largest output (the kernel's and the oracle's outputs are both rounded to
bf16, 3 mantissa bits fewer than fp16).
Heads are independent, so full-size runs are checked against the oracle on a
subset of (batch, head) pairs plus size-independent properties on all heads.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import kda_chunkwise_ref, kda_recurrent_ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
O_TOL = 2e-3
S_TOL = 1e-3


def max_abs(a, b):
    return (a.detach().double().cpu() - b.detach().double().cpu()).abs().max().item()


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm()).item()


@pytest.fixture(scope="module")
def wl(kda_pkg):
    import importlib
    return importlib.import_module("kimi_linear_amd.workloads")


def to_dev(inp):
    return {n: (t.to(DEV) if t is not None else None) for n, t in inp.items()}


def to_cpu(inp):
    return {n: (t.cpu() if t is not None else None) for n, t in inp.items()}


def run_chunkwise(pkg, inp, chunk, state_dtype=torch.float32):
    with torch.no_grad():
        return pkg.kda_chunkwise(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"],
                                 initial_state=inp["state"], chunk_size=chunk,
                                 state_dtype=state_dtype)


def ref_chunkwise(inp, chunk, state_dtype=torch.float32):
    return kda_chunkwise_ref(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"],
                             initial_state=inp["state"], chunk_size=chunk, state_dtype=state_dtype)


def run_recurrent(pkg, inp, state_dtype=torch.float32):
    with torch.no_grad():
        return pkg.kda_recurrent(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"],
                                 state=inp["state"], state_dtype=state_dtype)


def ref_recurrent(inp, state_dtype=torch.float32):
    return kda_recurrent_ref(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"],
                             state=inp["state"], state_dtype=state_dtype)


def report(tag, eo, es):
    print(f"[{tag}] o max-abs {eo:.3e}  state rel {es:.3e}", flush=True)


def o_bar(dtype, o_ref):
    """The output bar: O_TOL, plus one bf16 ulp of the largest output for bf16
    (two values rounded to bf16 from nearby fp32 values differ by at most one
    ulp, <= 2^-7 of their magnitude)."""
    return O_TOL + (2.0 ** -7 * float(o_ref.float().abs().max()) if dtype == torch.bfloat16 else 0.0)


# ----------------------------------------------------------------- configuration 0
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_config0_recurrent(kda_pkg, wl, dtype):
    inp = wl.make_inputs(1, 256, 2, 64, 64, seed=0, qkv_dtype=dtype)
    o, s = run_recurrent(kda_pkg, to_dev(inp))
    o_ref, s_ref = ref_recurrent(inp)
    eo, es = max_abs(o, o_ref), rel(s, s_ref)
    report(f"cfg0 recurrent {dtype}", eo, es)
    assert o.dtype == dtype and s.dtype == torch.float32
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert eo <= tol and es <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_config0_chunkwise(kda_pkg, wl, dtype):
    inp = wl.make_inputs(1, 256, 2, 64, 64, seed=0, qkv_dtype=dtype)
    o, s = run_chunkwise(kda_pkg, to_dev(inp), 64)
    o_ref, s_ref = ref_chunkwise(inp, 64)
    eo, es = max_abs(o, o_ref), rel(s, s_ref)
    report(f"cfg0 chunkwise {dtype}", eo, es)
    assert o.dtype == dtype
    if dtype == torch.float32:
        # fp32 activations are computed in fp32 throughout, like the reference's fp32 path
        assert eo <= 1e-5 and es <= 1e-5
    else:
        assert eo <= o_bar(dtype, o_ref) and es <= S_TOL


@pytest.mark.parametrize("big", ["state", "v"])
def test_chunkwise_fp32_wide_range(kda_pkg, wl, big):
    """fp32 inputs far outside the fp16 range (an initial state of order 1e6, or
    v of order 1e5) keep fp32 accuracy: relative errors <= 1e-5."""
    print(f"chunkwise fp32 wide range: large {big}", flush=True)
    inp = wl.make_inputs(2, 192, 2, 128, 64, seed=21, qkv_dtype=torch.float32, state_std=0.02)
    if big == "state":
        inp["state"] = inp["state"] * 5e7                      # |S| ~ 1e6
    else:
        inp["v"] = inp["v"] * 1e5
    o, s = run_chunkwise(kda_pkg, to_dev(inp), 64)
    o_ref, s_ref = ref_chunkwise(inp, 64)
    assert torch.isfinite(o).all() and torch.isfinite(s).all()
    eo = max_abs(o, o_ref) / o_ref.abs().max().item()
    es = rel(s, s_ref)
    report(f"fp32 wide range ({big}), o max-abs relative", eo, es)
    assert eo <= 1e-5 and es <= 1e-5


@pytest.mark.parametrize("big", ["state", "v"])
def test_chunkwise_bf16_wide_range(kda_pkg, wl, big):
    """bf16 inputs far outside the fp16 range: an initial state of order 1e6 or
    v of order 1e5 (the reference computes bf16 in fp32, kda.py:116).  The
    pipeline's fp16 operands see the state and values scaled by a power of two
    per consumer wave; outputs within the bf16 bar relative to their
    magnitude, the state within 1e-3."""
    print(f"chunkwise bf16 wide range: large {big}", flush=True)
    inp = wl.make_inputs(2, 192, 4, 128, 128, seed=23, qkv_dtype=torch.bfloat16, state_std=0.02)
    if big == "state":
        inp["state"] = inp["state"] * 5e7                      # |S| ~ 1e6
    else:
        inp["v"] = (inp["v"].float() * 1e5).to(torch.bfloat16)
    o, s = run_chunkwise(kda_pkg, to_dev(inp), 64)
    o_ref, s_ref = ref_chunkwise(inp, 64)
    assert torch.isfinite(o.float()).all() and torch.isfinite(s).all()
    scale = float(o_ref.float().abs().max())
    eo = max_abs(o, o_ref) / scale
    es = rel(s, s_ref)
    report(f"bf16 wide range ({big}), o max-abs relative to max|o| {scale:.1e}", eo, es)
    assert eo <= 2.0 ** -7 + O_TOL and es <= S_TOL


def test_config0_chunkwise_equals_recurrent_gpu(kda_pkg, wl):
    inp = to_dev(wl.make_inputs(1, 256, 2, 64, 64, seed=0, qkv_dtype=torch.float16))
    o_c, s_c = run_chunkwise(kda_pkg, inp, 64)
    o_r, s_r = run_recurrent(kda_pkg, inp)
    eo, es = max_abs(o_c, o_r), rel(s_c, s_r)
    report("cfg0 chunkwise vs recurrent (both GPU)", eo, es)
    assert eo <= O_TOL and es <= S_TOL


# ----------------------------------------------------------------- configuration 1
@pytest.fixture(scope="module")
def cfg1(wl):
    return wl.make_inputs(8, 4096, 16, 128, 128, device=DEV, seed=1, qkv_dtype=torch.float16)


def test_config1_chunkwise_vs_oracle(kda_pkg, wl, cfg1):
    o, s = run_chunkwise(kda_pkg, cfg1, 64)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(s).all()
    for b, h in ((0, 0), (3, 7), (7, 15)):
        sub = to_cpu(wl.slice_heads(cfg1, slice(b, b + 1), slice(h, h + 1)))
        o_ref, s_ref = ref_chunkwise(sub, 64)
        eo = max_abs(o[b:b + 1, :, h:h + 1], o_ref)
        es = rel(s[b:b + 1, h:h + 1], s_ref)
        report(f"cfg1 chunkwise b={b} h={h}", eo, es)
        assert eo <= O_TOL and es <= S_TOL


def test_config1_chunkwise_vs_gpu_recurrent_all_heads(kda_pkg, cfg1):
    # size-independent property on every head: two different algorithms agree
    o_c, s_c = run_chunkwise(kda_pkg, cfg1, 64)
    o_r, s_r = run_recurrent(kda_pkg, cfg1)
    eo, es = max_abs(o_c, o_r), rel(s_c, s_r)
    report("cfg1 chunkwise vs recurrent, all heads", eo, es)
    assert eo <= O_TOL and es <= S_TOL


def test_config1_chunk_size_invariance(kda_pkg, cfg1):
    o64, s64 = run_chunkwise(kda_pkg, cfg1, 64)
    o128, s128 = run_chunkwise(kda_pkg, cfg1, 128)
    # the kernel's internal chunk does not depend on chunk_size: bit-identical
    assert torch.equal(o64, o128) and torch.equal(s64, s128)


# ----------------------------------------------------------------- configuration 2
@pytest.mark.parametrize("B,H,T", [(4, 16, 512), (2, 8, 128), (6, 16, 256)])
def test_chunkwise_mid_head_counts(kda_pkg, wl, B, H, T):
    """64, 16 and 96 (batch, head) chains: the launch picks the column tile by
    rounds of workgroups, the 64-column one on a tie (one round at 64, 16 and
    96 chains: 128, 32 and 192 workgroups); every head against the oracle."""
    print(f"chunkwise B={B} H={H} T={T} K=V=128 fp16", flush=True)
    inp = wl.make_inputs(B, T, H, 128, 128, seed=B * 100 + H, qkv_dtype=torch.float16, state_std=0.02)
    o, s = run_chunkwise(kda_pkg, to_dev(inp), 64)
    o_ref, s_ref = ref_chunkwise(inp, 64)
    eo, es = max_abs(o, o_ref), rel(s, s_ref)
    report(f"mid heads B={B} H={H}", eo, es)
    assert eo <= O_TOL and es <= S_TOL


@pytest.mark.parametrize("K,dtype", [(128, torch.float16), (64, torch.bfloat16), (32, torch.float16)])
def test_chunkwise_many_heads_wide_tiles(kda_pkg, wl, K, dtype):
    """More 64-column tiles than CUs (3 x 64 heads x V=128): 128-column
    workgroups whose consumer waves own two 16-column groups.  Every column's
    arithmetic is the narrower kernel's, so one sequence run alone (64 heads,
    64-column tiles) must give the same bits; two heads are checked against
    the oracle."""
    B, T, H, V = 3, 96, 64, 128
    print(f"chunkwise wide tiles B={B} H={H} T={T} K={K} V={V} {dtype}", flush=True)
    inp = to_dev(wl.make_inputs(B, T, H, K, V, seed=K, qkv_dtype=dtype, state_std=0.02))
    o, s = run_chunkwise(kda_pkg, inp, 32)
    one = {n: (t[1:2] if t is not None else None) for n, t in inp.items()}
    o1, s1 = run_chunkwise(kda_pkg, one, 32)
    assert torch.equal(o[1:2], o1) and torch.equal(s[1:2], s1)
    sub = to_cpu(wl.slice_heads(inp, slice(2, 3), slice(5, 64, 50)))
    o_ref, s_ref = ref_chunkwise(sub, 32)
    eo, es = max_abs(o[2:3, :, 5:64:50], o_ref), rel(s[2:3, 5:64:50], s_ref)
    report(f"wide tiles K={K} {dtype}", eo, es)
    assert eo <= o_bar(dtype, o_ref) and es <= S_TOL


@pytest.mark.parametrize("V", [128, 256])
def test_recurrent_k256(kda_pkg, wl, V):
    """Head dim K = 256 (16 state columns a wave): fp32 recurrence vs the oracle."""
    print(f"recurrent K=256 V={V}", flush=True)
    inp = wl.make_inputs(2, 12, 3, 256, V, seed=V, qkv_dtype=torch.float32, state_std=0.02)
    o, s = run_recurrent(kda_pkg, to_dev(inp))
    o_ref, s_ref = ref_recurrent(inp)
    eo, es = max_abs(o, o_ref), rel(s, s_ref)
    report(f"recurrent K=256 V={V}", eo, es)
    assert eo <= 1e-5 and es <= 1e-5


def test_config2_decode_graph(kda_pkg, wl):
    B, H, K, V, steps = 64, 16, 128, 128, 512
    gen_inp = wl.make_inputs(B, steps, H, K, V, device=DEV, seed=2, qkv_dtype=torch.float16,
                             gate_dtype=torch.float16, state_std=0.02)
    s0 = gen_inp["state"]
    step_in = [{n: gen_inp[n][:, t:t + 1] for n in ("q", "k", "v", "g", "beta")}
               for t in range(steps)]
    # static buffers for the captured step: state ping-pong inside the graph
    st = s0.clone()
    xs = {n: torch.empty_like(step_in[0][n]) for n in step_in[0]}
    outs = torch.empty(steps, B, 1, H, V, device=DEV, dtype=torch.float16)

    def one_step(t_out):
        o, s_new = kda_pkg.kda_recurrent(xs["q"], xs["k"], xs["v"], xs["g"], xs["beta"],
                                         state=st, state_dtype=torch.float32)
        st.copy_(s_new)
        t_out.copy_(o)

    graph = torch.cuda.CUDAGraph()
    buf = torch.empty(B, 1, H, V, device=DEV, dtype=torch.float16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s), torch.no_grad():
        for n in xs:
            xs[n].copy_(step_in[0][n])
        one_step(buf)                                    # warm-up on a side stream
    torch.cuda.current_stream().wait_stream(s)
    st.copy_(s0)
    with torch.cuda.graph(graph), torch.no_grad():
        one_step(buf)
    st.copy_(s0)
    for t in range(steps):
        for n in xs:
            xs[n].copy_(step_in[t][n])
        graph.replay()
        outs[t].copy_(buf)
    torch.cuda.synchronize()
    # eager GPU run of the same 512 tokens in one call: identical arithmetic
    with torch.no_grad():
        o_all, s_all = kda_pkg.kda_recurrent(gen_inp["q"], gen_inp["k"], gen_inp["v"],
                                             gen_inp["g"], gen_inp["beta"], state=s0,
                                             state_dtype=torch.float32)
    graph_o = outs.squeeze(2).transpose(0, 1)            # [B, steps, H, V]
    assert torch.equal(graph_o, o_all) and torch.equal(st, s_all)
    # step-by-step oracle on a subset of batch rows (all heads)
    for b in (0, 63):
        sub = to_cpu(wl.slice_heads(gen_inp, slice(b, b + 1), slice(0, H)))
        o_ref, s_ref = ref_recurrent(sub)
        eo = max_abs(graph_o[b:b + 1], o_ref)
        es = rel(st[b:b + 1], s_ref)
        report(f"cfg2 512-step decode b={b}", eo, es)
        assert eo <= O_TOL and es <= 1e-5


@pytest.mark.parametrize("in_place", [False, True])
def test_config2_decode_512_steps_in_one_graph(kda_pkg, wl, in_place):
    """Configuration 2 as it is timed: 512 consecutive B=64 decode steps
    captured in ONE hipGraph (each step a fresh state tensor, as the
    reference's API returns it, or the state updated in place), every step's
    output kept; replayed twice.  Every step's o and the final state against
    the oracle's token recurrence (batch rows 0 and 63, all heads), and the
    whole replay against one eager call over the 512 tokens."""
    B, H, K, V, steps = 64, 16, 128, 128, 512
    print(f"cfg2 512 steps in one graph, in_place={in_place}", flush=True)
    inp = wl.make_inputs(B, steps, H, K, V, device=DEV, seed=2, qkv_dtype=torch.float16,
                         gate_dtype=torch.float16, state_std=0.02)
    xs = [inp[n] for n in ("q", "k", "v", "g", "beta")]
    st = inp["state"].clone()
    outs = torch.empty(B, steps, H, V, device=DEV, dtype=torch.float16)
    holder = {}

    def run_all(s_in):
        cur = s_in
        for t in range(steps):
            o, cur = kda_pkg.kda_recurrent(*[a[:, t:t + 1] for a in xs], state=cur, state_dtype=torch.float32,
                                           state_out=cur if in_place else None)
            outs[:, t:t + 1].copy_(o)
        holder["final"] = cur

    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            run_all(st)                                    # warm-up on a side stream
        torch.cuda.current_stream().wait_stream(side)
        st.copy_(inp["state"])
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run_all(st)
        final = holder["final"]
        o_all, s_all = kda_pkg.kda_recurrent(*xs, state=inp["state"], state_dtype=torch.float32)
        for rep in range(2):
            st.copy_(inp["state"])
            outs.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(outs, o_all) and torch.equal(final, s_all), rep
    for b in (0, 63):
        sub = to_cpu(wl.slice_heads(inp, slice(b, b + 1), slice(0, H)))
        o_ref, s_ref = ref_recurrent(sub)
        per_step = (outs[b:b + 1].double().cpu() - o_ref.double()).abs().amax(dim=(0, 2, 3))
        es = rel(final[b:b + 1], s_ref)
        report(f"cfg2 one-graph decode b={b} (worst step {int(per_step.argmax())})", per_step.max().item(), es)
        assert per_step.max().item() <= O_TOL and es <= 1e-5
    del graph


# ----------------------------------------------------------------- configuration 3
def test_config3_long_context_state(kda_pkg, wl):
    inp = wl.make_inputs(1, 32768, 16, 128, 128, device=DEV, seed=3, qkv_dtype=torch.float16,
                         a_log_range=(math.log(4.0), math.log(64.0)), state_std=0.02)
    o, s = run_chunkwise(kda_pkg, inp, 64)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(s).all()
    sub = to_cpu(wl.slice_heads(inp, slice(0, 1), slice(0, 16, 5)))
    o_ref, s_ref = ref_chunkwise(sub, 64)
    eo = max_abs(o[:, :, 0:16:5], o_ref)
    es = rel(s[:, 0:16:5], s_ref)
    report("cfg3 long context (heads 0,5,10,15)", eo, es)
    assert eo <= O_TOL and es <= S_TOL


# ----------------------------------------------------------------- edge cases
@pytest.mark.parametrize("T,chunk", [(40, 40), (16, 16), (5, 5), (1, 1), (200, 8)])
def test_ragged_lengths(kda_pkg, wl, T, chunk):
    inp = wl.make_inputs(2, T, 3, 64, 64, seed=4, qkv_dtype=torch.float16, state_std=0.02)
    o, s = run_chunkwise(kda_pkg, to_dev(inp), chunk)
    o_ref, s_ref = ref_chunkwise(inp, chunk)
    eo, es = max_abs(o, o_ref), rel(s, s_ref)
    report(f"ragged T={T} C={chunk}", eo, es)
    assert eo <= O_TOL and es <= S_TOL


def test_empty_inputs(kda_pkg, wl):
    inp = to_dev(wl.make_inputs(2, 0, 3, 64, 64, seed=5, qkv_dtype=torch.float16, state_std=0.02))
    o, s = run_chunkwise(kda_pkg, inp, 64)
    assert o.shape == (2, 0, 3, 64) and torch.equal(s, inp["state"])
    o, s = run_recurrent(kda_pkg, inp, state_dtype=torch.float16)
    assert s.dtype == torch.float16 and torch.equal(s, inp["state"].half())
    inp0 = to_dev(wl.make_inputs(0, 16, 3, 64, 64, seed=5, qkv_dtype=torch.float16))
    o, s = run_chunkwise(kda_pkg, inp0, 16)
    assert o.shape == (0, 16, 3, 64) and s.shape == (0, 3, 64, 64)


def test_strided_body_slice_and_dtypes(kda_pkg, wl):
    # the KDA layer passes q[:, :body] views of [B, T_full, H, D] projections
    inp = wl.make_inputs(2, 72, 4, 128, 128, seed=6, qkv_dtype=torch.float16,
                         gate_dtype=torch.float16, state_std=0.02, state_dtype=torch.float16)
    dev = to_dev(inp)
    body = {n: (t[:, :64] if n != "state" else t) for n, t in dev.items()}
    o, s = run_chunkwise(kda_pkg, body, 64, state_dtype=None)
    assert o.dtype == torch.float16 and s.dtype == torch.float16
    ref = {n: (t[:, :64] if n != "state" else t) for n, t in inp.items()}
    o_ref, s_ref = ref_chunkwise(ref, 64, state_dtype=torch.float32)
    eo, es = max_abs(o, o_ref), rel(s.float(), s_ref)
    report("strided body, fp16 gates/state", eo, es)
    assert eo <= O_TOL and es <= 2e-3        # fp16 state rounding adds ~5e-4
    # the tail through the recurrence, chained through the state
    tail = {n: (t[:, 64:] if n != "state" else s.float()) for n, t in dev.items()}
    o2, s2 = run_recurrent(kda_pkg, tail)
    ref_tail = {n: (t[:, 64:] if n != "state" else s_ref) for n, t in inp.items()}
    o2_ref, s2_ref = ref_recurrent(ref_tail)
    assert max_abs(o2, o2_ref) <= O_TOL and rel(s2, s2_ref) <= 2e-3


def test_broadcast_inputs(kda_pkg, wl):
    # stride-0 (expanded) token dimensions: the wrapper copies them to
    # distinct rows; results equal those of the materialised tensors
    inp = to_dev(wl.make_inputs(1, 64, 2, 64, 64, seed=8, qkv_dtype=torch.float16, state_std=0.02))
    ex = dict(inp)
    ex["k"] = inp["k"][:, :1].expand(-1, 64, -1, -1)
    ex["beta"] = inp["beta"][:, :1].expand(-1, 64, -1)
    mat = dict(ex)
    mat["k"], mat["beta"] = ex["k"].contiguous(), ex["beta"].contiguous()
    o1, s1 = run_chunkwise(kda_pkg, ex, 16)
    o2, s2 = run_chunkwise(kda_pkg, mat, 16)
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


@pytest.mark.parametrize("K,V", [(32, 32), (64, 16), (128, 64), (32, 128)])
def test_head_dims(kda_pkg, wl, K, V):
    inp = wl.make_inputs(1, 48, 2, K, V, seed=7, qkv_dtype=torch.float16, state_std=0.02)
    o, s = run_chunkwise(kda_pkg, to_dev(inp), 16)
    o_ref, s_ref = ref_chunkwise(inp, 16)
    eo, es = max_abs(o, o_ref), rel(s, s_ref)
    report(f"chunkwise K={K} V={V}", eo, es)
    assert eo <= O_TOL and es <= S_TOL
    if V % 32 == 0:
        o, s = run_recurrent(kda_pkg, to_dev(inp))
        o_ref, s_ref = ref_recurrent(inp)
        assert max_abs(o, o_ref) <= O_TOL and rel(s, s_ref) <= 1e-5


def test_recurrent_fp16_clamp(kda_pkg, wl):
    inp = wl.make_inputs(1, 4, 2, 64, 64, seed=8, qkv_dtype=torch.float16)
    inp["state"] = torch.full((1, 2, 64, 64), 1.0e7)     # |o| ~ 1e6 before the clamp
    o, _ = run_recurrent(kda_pkg, to_dev(inp))
    o_ref, _ = ref_recurrent(inp)
    o = o.cpu().float()
    o_ref = o_ref.float()
    clamped = o_ref.abs() == 60000.0
    assert clamped.float().mean().item() > 0.5
    assert torch.equal(o[clamped], o_ref[clamped])
    assert o.abs().max().item() == 60000.0
    rest = ~clamped
    assert ((o[rest] - o_ref[rest]).abs() <= 1e-3 * o_ref[rest].abs() + 1.0).all()


def test_inputs_not_mutated(kda_pkg, wl):
    inp = to_dev(wl.make_inputs(1, 32, 2, 64, 64, seed=9, qkv_dtype=torch.float16, state_std=0.02))
    before = {n: t.clone() for n, t in inp.items()}
    run_chunkwise(kda_pkg, inp, 16)
    run_recurrent(kda_pkg, inp)
    for n in inp:
        assert torch.equal(inp[n], before[n]), n


def test_chunkwise_graph_replays(kda_pkg, wl):
    inp = to_dev(wl.make_inputs(2, 256, 4, 128, 128, seed=10, qkv_dtype=torch.float16,
                                state_std=0.02))
    eager_o, eager_s = run_chunkwise(kda_pkg, inp, 64)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run_chunkwise(kda_pkg, inp, 64)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_o, g_s = run_chunkwise(kda_pkg, inp, 64)
    for _ in range(3):
        g_o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(g_o, eager_o) and torch.equal(g_s, eager_s)


def test_grad_inputs_rejected(kda_pkg, wl):
    """Under autograd the recurrence returns a new state (no state_out) and
    needs a head size the native backward takes; its gradients are checked in
    test_gpu_backward.py."""
    inp = to_dev(wl.make_inputs(1, 16, 1, 64, 64, seed=11, qkv_dtype=torch.float32))
    q = inp["q"].clone().requires_grad_(True)
    s_out = torch.empty(1, 1, 64, 64, device=q.device)
    with pytest.raises(kda_pkg.KdaError, match="in-place"):
        kda_pkg.kda_recurrent(q, inp["k"], inp["v"], inp["g"], inp["beta"], state_out=s_out)
    big = to_dev(wl.make_inputs(1, 4, 1, 256, 64, seed=12, qkv_dtype=torch.float32))
    with pytest.raises(kda_pkg.KdaError, match="backward supports"):
        kda_pkg.kda_recurrent(big["q"].clone().requires_grad_(True), big["k"], big["v"], big["g"], big["beta"])
