"""GPU tests of the in-place decode state and the hipGraph decoder over a stack
of KDA layers: every graph replay against the eager step-by-step layers (with
eager work and synchronisations between the replays), and the whole decoded
sequence against the layer oracle."""

from __future__ import annotations

import pytest
import torch

from oracle import kda_recurrent_ref
from oracle.kda_layer_oracle import kda_layer_ref, make_layer_params

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm()).item()


@pytest.fixture(scope="module")
def wl(kda_pkg):
    import importlib
    return importlib.import_module("kimi_linear_amd.workloads")


# ----------------------------------------------------------------- in-place kernel state
def test_recurrent_in_place_state(kda_pkg, wl):
    inp = wl.make_inputs(4, 3, 2, 128, 128, seed=11, qkv_dtype=torch.float16)
    st0 = torch.randn(4, 2, 128, 128, generator=torch.Generator().manual_seed(12)) * 0.02
    d = {n: t.to(DEV) for n, t in inp.items() if t is not None}
    with torch.no_grad():
        o_ref, s_ref = kda_pkg.kda_recurrent(d["q"], d["k"], d["v"], d["g"], d["beta"], state=st0.to(DEV),
                                             state_dtype=torch.float32)
        s = st0.to(DEV)
        o, s_ret = kda_pkg.kda_recurrent(d["q"], d["k"], d["v"], d["g"], d["beta"], state=s,
                                         state_dtype=torch.float32, state_out=s)
        torch.cuda.synchronize()
    assert s_ret.data_ptr() == s.data_ptr()
    assert torch.equal(o, o_ref) and torch.equal(s, s_ref)
    # a separate output buffer leaves the input alone
    s_in = st0.to(DEV)
    s_out = torch.empty_like(s_in)
    with torch.no_grad():
        kda_pkg.kda_recurrent(d["q"], d["k"], d["v"], d["g"], d["beta"], state=s_in, state_out=s_out,
                              state_dtype=torch.float32)
    assert torch.equal(s_in.cpu(), st0) and torch.equal(s_out, s_ref)
    o_cpu, s_cpu = kda_recurrent_ref(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], state=st0,
                                     state_dtype=torch.float32)
    assert rel(s, s_cpu) <= 1e-3 and (o.double().cpu() - o_cpu.double()).abs().max().item() <= 2e-3


def test_recurrent_state_out_errors(kda_pkg, wl):
    inp = wl.make_inputs(1, 1, 2, 64, 64, seed=13, qkv_dtype=torch.float16)
    d = {n: t.to(DEV) for n, t in inp.items() if t is not None}
    big = torch.zeros(2 * 2 * 64 * 64 + 64, device=DEV)
    s = big[:2 * 64 * 64].view(1, 2, 64, 64)
    shifted = big[64:64 + 2 * 64 * 64].view(1, 2, 64, 64)
    with torch.no_grad():
        with pytest.raises(kda_pkg.KdaError, match="overlaps"):
            kda_pkg.kda_recurrent(d["q"], d["k"], d["v"], d["g"], d["beta"], state=s, state_out=shifted,
                                  state_dtype=torch.float32)
        with pytest.raises(kda_pkg.KdaError, match="dtype"):
            kda_pkg.kda_recurrent(d["q"], d["k"], d["v"], d["g"], d["beta"], state=s,
                                  state_out=torch.empty(1, 2, 64, 64, device=DEV, dtype=torch.float16),
                                  state_dtype=torch.float32)
        with pytest.raises(kda_pkg.KdaError, match="contiguous"):
            kda_pkg.kda_recurrent(d["q"], d["k"], d["v"], d["g"], d["beta"], state=s,
                                  state_out=torch.empty(1, 2, 64, 64, device=DEV).transpose(2, 3),
                                  state_dtype=torch.float32)


def test_in_place_step_graph_replays(kda_pkg, wl):
    """One captured in-place decode step replayed 6 times chains the state
    exactly like 6 eager steps (eager work and a sync between replays)."""
    B, H, K, V = 8, 4, 128, 128
    steps = [wl.make_inputs(B, 1, H, K, V, seed=20 + i, qkv_dtype=torch.float16) for i in range(6)]
    st0 = torch.randn(B, H, K, V, generator=torch.Generator().manual_seed(19)) * 0.02
    static_in = {n: steps[0][n].to(DEV) for n in ("q", "k", "v", "g", "beta")}
    state = st0.to(DEV)
    out = {}

    def step():
        o, _ = kda_pkg.kda_recurrent(static_in["q"], static_in["k"], static_in["v"], static_in["g"],
                                     static_in["beta"], state=state, state_dtype=torch.float32,
                                     state_out=state)
        out["o"] = o

    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        state.copy_(st0.to(DEV))
        eager_s = st0.to(DEV)
        for i, inp in enumerate(steps):
            for n in static_in:
                static_in[n].copy_(inp[n].to(DEV))
            graph.replay()
            torch.cuda.synchronize()
            o_e, eager_s = kda_pkg.kda_recurrent(*(inp[n].to(DEV) for n in ("q", "k", "v", "g", "beta")),
                                                 state=eager_s, state_dtype=torch.float32)
            torch.cuda.synchronize()
            assert torch.equal(out["o"], o_e), f"replay {i}"
            assert torch.equal(state, eager_s), f"replay {i}"


# ----------------------------------------------------------------- graph decoder
def make_stack(pkg, n_layers, dtype, seed):
    cfg = pkg.linear_attn_config(hidden_size=256, num_heads=2, gate_low_rank=64, output_gate_low_rank=64)
    layers, params = [], []
    for i in range(n_layers):
        m = pkg.KimiDeltaAttention(cfg)
        m.load_state_dict(make_layer_params(cfg, seed=seed + i))
        m = m.to(device=DEV, dtype=dtype).eval()
        layers.append(m)
        params.append({n: t.detach().float().cpu() for n, t in m.state_dict().items()})
    return cfg, layers, params


def oracle_stack(cfg, params, x):
    h = x.float()
    for p in params:
        h = h + kda_layer_ref(p, cfg, h)
    return h


def test_graphed_decoder_vs_eager_and_oracle(kda_pkg):
    from kimi_linear_amd.graph_decode import KdaGraphedDecoder

    B, S, n_steps = 3, 40, 10
    cfg, layers, params = make_stack(kda_pkg, 2, torch.float16, seed=30)
    g = torch.Generator().manual_seed(31)
    x = (torch.randn(B, S + n_steps, 256, generator=g)).half()
    xd = x.to(DEV)
    dec = KdaGraphedDecoder(layers)
    with torch.no_grad():
        h0 = dec.prefill(xd[:, :S])
        # eager reference: the same layers, step by step through forward(use_cache=True)
        states = [None] * len(layers)
        h = xd[:, :S]
        for i, layer in enumerate(layers):
            out, states[i] = layer(h, state=states[i], use_cache=True)
            h = h + out
        assert torch.equal(h0, h[:, -1])
        got, want = [], []
        for t in range(S, S + n_steps):
            y = dec.step(xd[:, t:t + 1]).clone()
            torch.cuda.synchronize()
            h = xd[:, t:t + 1]
            for i, layer in enumerate(layers):
                out, states[i] = layer(h, state=states[i], use_cache=True)
                h = h + out
            torch.cuda.synchronize()
            e = rel(y, h[:, -1])
            print(f"[graph decode step {t}] rel vs eager {e:.3e}", flush=True)
            assert e <= 1e-3
            got.append(y)
            want.append(h[:, -1])
        for st, ref in zip(dec.static_states, states):
            assert rel(st["recurrent"], ref["recurrent"]) <= 1e-3
            for n in ("q", "k", "v"):
                assert torch.equal(st["conv"][n], ref["conv"][n])
    full = oracle_stack(cfg, params, x)
    e = rel(torch.stack(got, 1), full[:, S:])
    print(f"[graph decode] rel vs oracle {e:.3e}", flush=True)
    assert e <= 1e-2


def test_graphed_decoder_reprefill_reuses_graph(kda_pkg):
    from kimi_linear_amd.graph_decode import KdaGraphedDecoder

    B = 2
    cfg, layers, params = make_stack(kda_pkg, 1, torch.float16, seed=40)
    dec = KdaGraphedDecoder(layers)
    g = torch.Generator().manual_seed(41)
    first = None
    for prompt_len in (24, 70):
        x = torch.randn(B, prompt_len + 4, 256, generator=g).half()
        xd = x.to(DEV)
        with torch.no_grad():
            dec.prefill(xd[:, :prompt_len])
            first = first or dec.graph
            assert dec.graph is first            # same batch size: no re-capture
            ys = [dec.step(xd[:, t:t + 1]).clone() for t in range(prompt_len, prompt_len + 4)]
        full = oracle_stack(cfg, params, x)
        e = rel(torch.stack(ys, 1), full[:, prompt_len:])
        print(f"[graph decode re-prefill {prompt_len}] rel vs oracle {e:.3e}", flush=True)
        assert e <= 1e-2


def test_graphed_decoder_follows_weight_updates(kda_pkg):
    """Weights loaded in place after capture (load_state_dict) reach the replayed
    step: the next prefill refills the fused projection weight in its own buffer
    (the captured GEMM keeps reading valid memory, no recapture), and
    refresh_weights() does the same between two steps of one generation."""
    from kimi_linear_amd.graph_decode import KdaGraphedDecoder

    B = 2
    cfg, layers, _ = make_stack(kda_pkg, 1, torch.float16, seed=50)
    dec = KdaGraphedDecoder(layers)
    g = torch.Generator().manual_seed(51)
    x = torch.randn(B, 30, 256, generator=g).half().to(DEV)
    new_params = make_layer_params(cfg, seed=52)
    with torch.no_grad():
        dec.prefill(x[:, :24])
        graph = dec.graph
        dec.step(x[:, 24:25])
        layers[0].load_state_dict(new_params)                  # copy_ into the live parameters
        dec.prefill(x[:, :24])
        assert dec.graph is graph                              # the fused weight stayed in place
        ys = [dec.step(x[:, t:t + 1]).clone() for t in range(24, 27)]
        fresh_cfg, fresh, fresh_params = make_stack(kda_pkg, 1, torch.float16, seed=52)
        ref_dec = KdaGraphedDecoder(fresh)
        ref_dec.prefill(x[:, :24])
        want = [ref_dec.step(x[:, t:t + 1]).clone() for t in range(24, 27)]
        for a, b in zip(ys, want):
            assert torch.equal(a, b)
        # an update between two steps of one generation, then refresh_weights()
        layers[0].load_state_dict(make_layer_params(cfg, seed=50))
        fresh[0].load_state_dict(make_layer_params(cfg, seed=50))
        dec.refresh_weights()
        ref_dec.refresh_weights()
        a = dec.step(x[:, 27:28]).clone()
        b = ref_dec.step(x[:, 27:28]).clone()
        assert torch.equal(a, b)
