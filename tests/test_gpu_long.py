"""GPU parity of the split long-sequence path (kda_chunkwise_long_fwd).

A long sequence with few (batch, head) chains is cut into segments that run
in parallel: per segment the state from zero and the K x K transition, a
sequential composition of the segments in fp32, then the outputs from the
true initial states -- with few chains (the first pass in one round of
workgroups) as the outputs from a zero state, which the first pass keeps in
fp32, plus their initial-state coefficients (the transition columns'
outputs) times the composed initial states.  The result is the same function as one pass, rounded
differently: against the oracle at the core bars (fp16 inputs: o max-abs
<= 2e-3, state relative error <= 1e-3), against one pass to 1e-3, and the
transitions are checked on their own by a zero-input case (the state then
only decays and mixes: every segment's Phi applied to S_0 must equal the
one-pass state).
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from oracle import kda_chunkwise_ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
O_TOL = 2e-3
S_TOL = 1e-3


@pytest.fixture(scope="module")
def wl(kda_pkg):
    import importlib
    return importlib.import_module("kimi_linear_amd.workloads")


@pytest.fixture(scope="module")
def native(kda_pkg):
    import importlib
    mod = importlib.import_module("kimi_linear_amd._native")
    mod.load()
    return mod


def max_abs(a, b):
    return (a.detach().double().cpu() - b.detach().double().cpu()).abs().max().item()


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm()).item()


def long_call(native, inp, segments, chunk=64):
    """kda_chunkwise_long_fwd through the C ABI (fp32 state out)."""
    q, k, v, g, beta, s0 = inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["state"]
    B, T, H, K = q.shape
    V = v.shape[-1]
    code = {torch.float32: native.DTYPE_F32, torch.float16: native.DTYPE_F16, torch.bfloat16: native.DTYPE_BF16}
    o = torch.empty(B, T, H, V, device=DEV, dtype=v.dtype)
    s = torch.empty(B, H, K, V, device=DEV, dtype=torch.float32)
    a = native.KdaFwdArgs()
    a.B, a.T, a.H, a.K, a.V = B, T, H, K, V
    a.q, a.k, a.v, a.g, a.beta = (x.data_ptr() for x in (q, k, v, g, beta))
    for name, x in (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta)):
        setattr(a, name + "_stride", (ctypes.c_int64 * 3)(*x.stride()[:3]))
    a.qkv_dtype, a.g_dtype, a.beta_dtype = code[v.dtype], native.DTYPE_F32, native.DTYPE_F32
    a.state_in = s0.data_ptr() if s0 is not None else None
    a.state_in_dtype = native.DTYPE_F32
    a.state_out, a.state_out_dtype, a.o = s.data_ptr(), native.DTYPE_F32, o.data_ptr()
    a.scale, a.clamp_fp16_out, a.chunk_size = float(K) ** -0.5, 0, chunk
    lib = native.load()
    ws = torch.empty(max(int(lib.kda_chunkwise_long_workspace_size(B, T, H, K, V, segments)), 16),
                     device=DEV, dtype=torch.uint8)
    st = lib.kda_chunkwise_long_fwd(ctypes.byref(a), segments, ctypes.c_void_p(ws.data_ptr()),
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, native.status_str(st)
    return o, s


@pytest.mark.parametrize("decay", [1.0, 1e-3])
@pytest.mark.parametrize("K,dtype,segments", [(128, torch.float16, 4), (64, torch.float16, 8),
                                              (128, torch.bfloat16, 2)])
def test_long_split_matches_oracle_and_one_pass(kda_pkg, wl, native, K, dtype, segments, decay):
    """decay scales g: at 1 (the layer's distribution) a segment forgets its
    initial state entirely (Phi underflows to 0), at 1e-3 it keeps most of it
    and Phi is a full matrix (the delta rule mixes the channels)."""
    B, T, H, V = 2, 2048, 2, 128
    print(f"long split B={B} T={T} H={H} K={K} V={V} {dtype} segments={segments} decay x{decay}", flush=True)
    cpu = wl.make_inputs(B, T, H, K, V, seed=31 + K, qkv_dtype=dtype, state_std=0.02)
    cpu["g"] = cpu["g"] * decay
    inp = {n: (t.to(DEV) if t is not None else None) for n, t in cpu.items()}
    with torch.no_grad():
        o, s = long_call(native, inp, segments)
        o1, s1 = long_call(native, inp, 1)
    o_ref, s_ref = kda_chunkwise_ref(cpu["q"], cpu["k"], cpu["v"], cpu["g"], cpu["beta"],
                                     initial_state=cpu["state"], chunk_size=64, state_dtype=torch.float32)
    eo, es = max_abs(o, o_ref), rel(s, s_ref)
    d_o, d_s = rel(o, o1), rel(s, s1)
    print(f"  vs oracle: o max-abs {eo:.2e} state rel {es:.2e}; vs one pass: o {d_o:.2e} state {d_s:.2e}",
          flush=True)
    # bf16: one output ulp (2^-7 of the largest output) on top of the fp16 bars
    o_tol = O_TOL + (2.0 ** -7 * float(o_ref.float().abs().max()) if dtype == torch.bfloat16 else 0.0)
    assert eo <= o_tol and es <= S_TOL
    assert d_o <= (1e-3 if dtype == torch.float16 else 4e-3) and d_s <= 1e-3


def test_long_split_three_passes_at_many_chains(kda_pkg, wl, native):
    """64 heads in 4 segments: the first pass takes two rounds of 128-column
    workgroups, so the outputs come from the third pass over every chain from
    its true initial state (the cases above, with few chains, take the
    outputs from a zero state plus their initial-state coefficients times the
    composed initial states).  Against one pass and, on three heads, the
    oracle, with weak decays (each segment's initial state matters)."""
    B, T, H, K, V, segments = 1, 2048, 64, 128, 128, 4
    print(f"long split B={B} T={T} H={H} K={K} V={V} fp16 segments={segments} (three passes)", flush=True)
    cpu = wl.make_inputs(B, T, H, K, V, seed=61, qkv_dtype=torch.float16, state_std=0.02)
    cpu["g"] = cpu["g"] * 1e-3
    inp = {n: (t.to(DEV) if t is not None else None) for n, t in cpu.items()}
    with torch.no_grad():
        o, s = long_call(native, inp, segments)
        o1, s1 = long_call(native, inp, 1)
    d_o, d_s = rel(o, o1), rel(s, s1)
    sub = {n: (t[:, :, 0:64:31] if n != "state" else t[:, 0:64:31]) for n, t in cpu.items()}
    o_ref, s_ref = kda_chunkwise_ref(sub["q"], sub["k"], sub["v"], sub["g"], sub["beta"],
                                     initial_state=sub["state"], chunk_size=64, state_dtype=torch.float32)
    eo, es = max_abs(o[:, :, 0:64:31], o_ref), rel(s[:, 0:64:31], s_ref)
    print(f"  vs oracle: o max-abs {eo:.2e} state rel {es:.2e}; vs one pass: o {d_o:.2e} state {d_s:.2e}",
          flush=True)
    assert eo <= O_TOL and es <= S_TOL
    assert d_o <= 1e-3 and d_s <= 1e-3


def test_long_split_zero_inputs_carry_the_state(kda_pkg, wl, native):
    """v = 0 and k = 0: no write, the state only decays -- every segment's
    transition is then Diag(prod a) -- so the split state must be the product
    of all the decays times S_0 (weak decays keep it alive over 4096 tokens);
    the outputs (q~ E S, k = 0) must equal one pass's."""
    B, T, H, K, V = 1, 4096, 2, 128, 128
    cpu = wl.make_inputs(B, T, H, K, V, seed=41, qkv_dtype=torch.float16, state_std=1.0)
    cpu["k"] = torch.zeros_like(cpu["k"])
    cpu["v"] = torch.zeros_like(cpu["v"])
    cpu["g"] = cpu["g"] * 1e-3
    inp = {n: (t.to(DEV) if t is not None else None) for n, t in cpu.items()}
    with torch.no_grad():
        o, s = long_call(native, inp, 4)
        o1, _ = long_call(native, inp, 1)
    decay = torch.exp(cpu["g"].double().sum(1))                  # [B, H, K]
    want = cpu["state"].double() * decay[..., None]
    err = rel(s, want)
    print(f"long split zero inputs: state rel err {err:.2e}, o vs one pass {rel(o, o1):.2e}", flush=True)
    assert err <= 1e-4
    assert rel(o, o1) <= 1e-3


def test_wrapper_split_with_partial_last_chunks(kda_pkg, wl, native):
    """B=1 T=4160 H=16: the wrapper splits into 8 segments of 520 tokens, so
    every segment ends part-way through a 32-token chunk.  The rows past a
    segment's end must read as zero (not as the next segment's first tokens)
    in both the transition pass and the output pass: the wrapper's result
    against one pass and against the oracle on three heads."""
    kda = __import__("kimi_linear_amd.kda", fromlist=["long_segments"])
    B, T, H, K, V = 1, 4160, 16, 128, 128
    assert kda.long_segments(B, T, H, K, V, torch.float16) == 8 and (T // 8) % 32 != 0
    print(f"long split through the wrapper, B={B} T={T} H={H}: 8 segments of {T // 8} tokens", flush=True)
    cpu = wl.make_inputs(B, T, H, K, V, seed=51, qkv_dtype=torch.float16, state_std=0.02)
    cpu["g"] = cpu["g"] * 1e-3                      # weak decay: each segment's initial state matters
    inp = {n: (t.to(DEV) if t is not None else None) for n, t in cpu.items()}
    with torch.no_grad():
        o, s = kda_pkg.kda_chunkwise(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"],
                                     initial_state=inp["state"], chunk_size=64, state_dtype=torch.float32)
        o1, s1 = long_call(native, inp, 1)
    d_o, d_s = rel(o, o1), rel(s, s1)
    sub = {n: (t[:, :, 0:16:7] if n != "state" else t[:, 0:16:7]) for n, t in cpu.items()}
    o_ref, s_ref = kda_chunkwise_ref(sub["q"], sub["k"], sub["v"], sub["g"], sub["beta"],
                                     initial_state=sub["state"], chunk_size=64, state_dtype=torch.float32)
    eo, es = max_abs(o[:, :, 0:16:7], o_ref), rel(s[:, 0:16:7], s_ref)
    print(f"  vs oracle: o max-abs {eo:.2e} state rel {es:.2e}; vs one pass: o {d_o:.2e} state {d_s:.2e}",
          flush=True)
    assert eo <= O_TOL and es <= S_TOL
    assert d_o <= 1e-3 and d_s <= 1e-3


def test_wrapper_splits_the_config3_shape(kda_pkg):
    """The wrapper picks the split for one long sequence of 16 heads."""
    kda = __import__("kimi_linear_amd.kda", fromlist=["long_segments"])
    assert kda.long_segments(1, 32768, 16, 128, 128, torch.float16) == 8     # few-chain form
    assert kda.long_segments(1, 32768, 16, 128, 64, torch.float16) == 16     # V + K = 192: three passes
    assert kda.long_segments(1, 8192, 16, 128, 128, torch.float16) == 8
    assert kda.long_segments(8, 4096, 16, 128, 128, torch.float16) == 1
    assert kda.long_segments(1, 4096, 16, 128, 128, torch.float16) == 8
    assert kda.long_segments(2, 2048, 16, 128, 128, torch.float16) == 4
    assert kda.long_segments(3, 2048, 16, 128, 128, torch.float16) == 2
    assert kda.long_segments(4, 2048, 16, 128, 128, torch.float16) == 1     # the chains fill half the CUs
    assert kda.long_segments(1, 32768, 16, 128, 128, torch.float32) == 1
