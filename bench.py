"""Benchmark of the MI355X KDA core (one GPU).

A step is one ``kda_chunkwise`` forward over the 1.5B-config layer shape
(B=8, T=4096, H=16, dk=dv=128, chunk 64; fp16 q/k/v, fp32 g/beta, fp32 state
from zeros), inputs resident in HBM.  ``value`` is tokens/s (B*T per step).

Also reported on the same line:
* ``roofline`` of the chunkwise kernel: algorithmic HBM bytes per launch over
  the mean launch duration (HIP events around every timed launch);
* ``decode``: the B=64 recurrent decode step (fp32 state N(0, 0.02), fp16
  q/k/v/g/beta) as 512 chained steps captured in one hipGraph, per-step time,
  plus a variant rotating 5 independent state sets (320 MiB working set) so
  the state cannot stay resident in the 256 MB Infinity Cache, each both with
  a fresh state tensor per step (the reference API) and updated in place
  (``state_out=state``, as the graph decoder runs it);
* ``gated``: ``kda_chunkwise_gated`` at the same shape -- the layer's gate
  pre-processing formed in the kernel's loads from fp16 gk and beta logits
  (1282 instead of 1540 algorithmic bytes per token and head);
* ``long_context``: ``kda_chunkwise`` on one long sequence, B=1 T=32768 H=16
  (fp32 initial state, strong decay): 16 chains of 512 chunks each;
* ``layer``: the whole KDA layer at hidden 2048 (projections, short
  convolutions, norms and gates around the core): a B=4 T=2048 prefill and a
  graph-replayed B=64 decode token;
* ``cpu_baseline``: the CPU oracle (an op-for-op restatement of the
  reference's PyTorch algorithm) on a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 60] [--no-cpu]
"""

from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "KDA chunkwise fwd tokens/s @H16 d128 T4096 fp16; recurrent decode µs @B64"
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0

B1, T1, H1, D1, C1 = 8, 4096, 16, 128, 64
# algorithmic traffic per (token, head): q,k,v fp16 (768 B) + g fp32 (512 B) + beta (4 B)
# + o fp16 (256 B); per (sequence, head) the fp32 state is written once (S0 = 0 is not read).
CHUNK_BYTES = B1 * T1 * H1 * 1540 + B1 * H1 * D1 * D1 * 4
# the gated form reads gk and the beta logit in fp16: 3 x 256 + 256 + 2 + 256 B
GATED_BYTES = B1 * T1 * H1 * 1282 + B1 * H1 * D1 * D1 * 4
# causal flop count per (token, head): C (3K + 2V) + 6 K V
CHUNK_FLOPS = B1 * T1 * H1 * (C1 * (3 * D1 + 2 * D1) + 6 * D1 * D1)

B2, H2, STEPS2 = 64, 16, 512
# per decode step: fp32 state read + write, plus q,k,g,v (fp16) + beta (fp16) in and o (fp16) out
DECODE_BYTES = 2 * B2 * H2 * D1 * D1 * 4 + B2 * H2 * (4 * D1 * 2 + 2 + D1 * 2)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=60,
                   help="untimed steps first; the GPU clock takes ~20 ms of load to settle")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--decode-variant", choices=["all", "fresh", "in_place", "fresh_rot5", "in_place_rot5"],
                   default="all", help="with --only decode: time one variant (for kernel traces)")
    p.add_argument("--only", choices=["chunkwise", "gated", "long", "decode", "layer", "backward", "copy"],
                   default=None,
                   help="run one workload only (for profiling); 'copy' runs a plain 1 GiB "
                        "device copy used to calibrate the HBM byte counters")
    return p.parse_args()


def chunkwise_inputs(wl, torch):
    return wl.make_inputs(B1, T1, H1, D1, D1, device="cuda", seed=1, qkv_dtype=torch.float16)


def chunkwise_bench(pkg, wl, torch, steps, warmup, inp=None):
    inp = inp if inp is not None else chunkwise_inputs(wl, torch)
    args = (inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"])

    def step():
        return pkg.kda_chunkwise(*args, initial_state=None, chunk_size=C1,
                                 state_dtype=torch.float32)

    with torch.no_grad():
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
        t0 = time.perf_counter()
        for e0, e1 in ev:
            e0.record(stream)
            step()
            e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    launch_ms = sum(e0.elapsed_time(e1) for e0, e1 in ev) / steps
    return wall, launch_ms


def gated_bench(pkg, wl, torch, steps, warmup, inp=None):
    """kda_chunkwise_gated at the headline shape: fp16 q/k/v, fp16 gk and beta
    logits (the gate's pre-activations), fp32 A_log / dt_bias [H, K].  Returns
    the mean launch time in ms (HIP events around every timed launch)."""
    inp = inp if inp is not None else chunkwise_inputs(wl, torch)
    gen = torch.Generator(device="cuda").manual_seed(7)
    gk = torch.randn(B1, T1, H1, D1, device="cuda", generator=gen).half()
    logit = torch.randn(B1, T1, H1, device="cuda", generator=gen).half()
    a_log = torch.rand(H1, D1, device="cuda", generator=gen) * wl.LN16
    dt_bias = torch.randn(H1, D1, device="cuda", generator=gen) * 0.1

    def step():
        return pkg.kda_chunkwise_gated(inp["q"], inp["k"], inp["v"], gk, logit, a_log, dt_bias,
                                       chunk_size=C1, state_dtype=torch.float32)

    with torch.no_grad():
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
        for e0, e1 in ev:
            e0.record(stream)
            step()
            e1.record(stream)
        torch.cuda.synchronize()
    return sum(e0.elapsed_time(e1) for e0, e1 in ev) / steps


def long_context_bench(pkg, wl, torch, reps=3):
    """kda_chunkwise at B=1 T=32768 H=16 dk=dv=128 (fp16 q/k/v, fp32 g/beta,
    A_log ~ U(log 4, log 64), fp32 S0 ~ N(0, 0.02)); mean launch time in ms."""
    import math
    B3, T3 = 1, 32768
    inp = wl.make_inputs(B3, T3, H1, D1, D1, device="cuda", seed=3, qkv_dtype=torch.float16,
                         a_log_range=(math.log(4.0), math.log(64.0)), state_std=0.02)
    args = (inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"])
    with torch.no_grad():
        for _ in range(2):
            pkg.kda_chunkwise(*args, initial_state=inp["state"], chunk_size=C1, state_dtype=torch.float32)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            pkg.kda_chunkwise(*args, initial_state=inp["state"], chunk_size=C1, state_dtype=torch.float32)
        e1.record()
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    nbytes = B3 * T3 * H1 * 1540 + 2 * B3 * H1 * D1 * D1 * 4
    return {"workload": "kda_chunkwise, B=1 T=32768 H=16 dk=dv=128 chunk_size=64; fp16 q/k/v, fp32 g/beta "
                        "(A_log ~ U(log 4, log 64)), fp32 S0 ~ N(0, 0.02)",
            "ms": ms, "tokens_per_s": B3 * T3 / (ms * 1e-3), "algorithmic_bytes": nbytes,
            "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}


def decode_bench(pkg, wl, torch, n_sets, in_place=False):
    """512 chained decode steps in one hipGraph; returns us per step.

    ``n_sets`` independent state sets are stepped in turn (5 sets = 320 MiB,
    more than the Infinity Cache holds).  ``in_place``: each step overwrites
    its state (``state_out=state``, the graph decoder's form); otherwise each
    step returns a fresh state tensor, as the reference's API does."""
    inp = wl.make_inputs(B2, STEPS2, H2, D1, D1, device="cuda", seed=2,
                         qkv_dtype=torch.float16, gate_dtype=torch.float16, state_std=0.02)
    states = [inp["state"]] + [inp["state"].clone() for _ in range(n_sets - 1)]
    xs = [inp[n] for n in ("q", "k", "v", "g", "beta")]

    def run_all(sts):
        cur = list(sts)
        for t in range(STEPS2):
            c = t % n_sets
            x = [a[:, t:t + 1] for a in xs]
            _, cur[c] = pkg.kda_recurrent(*x, state=cur[c], state_dtype=torch.float32,
                                          state_out=cur[c] if in_place else None)
        return cur

    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            run_all(states)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run_all(states)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 5
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * STEPS2)
    del graph
    return us


def copy_bench(torch, n_sets=5):
    """A plain device copy of one decode state (64 MiB read + 64 MiB written)
    per step, n_sets buffer pairs in turn, 512 steps in one hipGraph: the
    bandwidth reference for the decode step."""
    n = B2 * H2 * D1 * D1
    src = [torch.randn(n, device="cuda") for _ in range(n_sets)]
    dst = [torch.empty_like(x) for x in src]

    def run_all():
        for t in range(STEPS2):
            dst[t % n_sets].copy_(src[t % n_sets])

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run_all()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_all()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 5
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * STEPS2)
    del graph
    return us


def layer_bench(pkg, torch, reps=10):
    """The whole KDA layer at hidden 2048 (16 heads of 128, fp16 weights N(0, 0.02),
    fp32 state): a B=4 T=2048 prefill forward, one training step (forward and
    backward to every parameter and x) at the same shape, and one
    graph-replayed decode token at B=64 (the layer's static state updated in
    place)."""
    from kimi_linear_amd.graph_decode import KdaGraphedDecoder

    cfg = pkg.linear_attn_config(hidden_size=2048, num_heads=16)
    torch.manual_seed(0)
    layer = pkg.KimiDeltaAttention(cfg)
    with torch.no_grad():
        for name, prm in layer.named_parameters():
            if name.endswith("weight") and prm.dim() >= 2:
                prm.normal_(0.0, 0.02)
    layer = layer.to(device="cuda", dtype=torch.float16).eval()
    x = torch.randn(4, 2048, 2048, device="cuda", dtype=torch.float16)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.no_grad():
        for _ in range(2):
            layer(x)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            layer(x)
        e1.record()
        torch.cuda.synchronize()
        prefill_ms = e0.elapsed_time(e1) / reps
        # a larger batch: 256 heads, where the layer runs the output epilogue
        # inside the chunk kernel (one workgroup per head)
        xb = torch.randn(16, 2048, 2048, device="cuda", dtype=torch.float16)
        for _ in range(2):
            layer(xb)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps // 2):
            layer(xb)
        e1.record()
        torch.cuda.synchronize()
        prefill16_ms = e0.elapsed_time(e1) / (reps // 2)
        del xb
        # one long prompt: 16 chains, where the core splits the sequence into
        # parallel segments
        xl = torch.randn(1, 16384, 2048, device="cuda", dtype=torch.float16)
        for _ in range(2):
            layer(xl)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps // 2):
            layer(xl)
        e1.record()
        torch.cuda.synchronize()
        prefill_long_ms = e0.elapsed_time(e1) / (reps // 2)
        del xl
    # training step: the differentiable path, gradients of every parameter and x
    xt = x.clone().requires_grad_()
    gout = torch.randn(4, 2048, 2048, device="cuda", dtype=torch.float16)
    for _ in range(2):
        layer(xt).backward(gout)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps // 2):
        layer.zero_grad(set_to_none=True)
        xt.grad = None
        layer(xt).backward(gout)
    e1.record()
    torch.cuda.synchronize()
    train_ms = e0.elapsed_time(e1) / (reps // 2)
    del xt, gout
    layer.zero_grad(set_to_none=True)
    with torch.no_grad():
        dec = KdaGraphedDecoder([layer])
        xd = torch.randn(64, 17, 2048, device="cuda", dtype=torch.float16)
        dec.prefill(xd[:, :16])
        tok = xd[:, 16:17]
        for _ in range(3):
            dec.step(tok)
        torch.cuda.synchronize()
        n = 100
        e0.record()
        for _ in range(n):
            dec.step(tok)
        e1.record()
        torch.cuda.synchronize()
        decode_us = e0.elapsed_time(e1) * 1e3 / n
    # the core the B=4 T=2048 prefill runs: kda_chunkwise_gated on the layer's
    # q, k, v and gate pre-activations (fp16), alone, HIP events around each launch
    with torch.no_grad():
        gen = torch.Generator(device="cuda").manual_seed(5)
        cq = torch.nn.functional.normalize(torch.randn(4, 2048, 16, 128, device="cuda", generator=gen), dim=-1).half()
        ck = torch.nn.functional.normalize(torch.randn(4, 2048, 16, 128, device="cuda", generator=gen), dim=-1).half()
        cv = torch.randn(4, 2048, 16, 128, device="cuda", generator=gen).half()
        cgk = torch.randn(4, 2048, 16, 128, device="cuda", generator=gen).half()
        cbl = torch.randn(4, 2048, 16, device="cuda", generator=gen).half()
        a_log, dt_bias = layer.A_log.detach().float(), layer.dt_bias.detach().float()
        core = lambda: pkg.kda_chunkwise_gated(cq, ck, cv, cgk, cbl, a_log, dt_bias,  # noqa: E731
                                               chunk_size=64, state_dtype=torch.float32)
        for _ in range(30):
            core()
        torch.cuda.synchronize()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for c0, c1 in evs:
            c0.record()
            core()
            c1.record()
        torch.cuda.synchronize()
        core_ms = sum(c0.elapsed_time(c1) for c0, c1 in evs) / reps
        del cq, ck, cv, cgk, cbl
    core_bytes = 4 * 2048 * 16 * 1282 + 4 * 16 * 128 * 128 * 4
    return {"workload": "KimiDeltaAttention hidden 2048, 16 heads x 128, fp16 weights, fp32 state",
            "core_B4_T2048_kernel_ms": core_ms,
            "core_B4_T2048_hbm_frac": core_bytes / (core_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "core_B4_T2048_note": "kda_chunkwise_gated alone at the prefill's shape (1282 B per token and head "
                                  "+ the fp32 state written), mean launch time from HIP events",
            "prefill_B4_T2048_ms": prefill_ms,
            "prefill_tokens_per_s": 4 * 2048 / (prefill_ms * 1e-3),
            "prefill_B16_T2048_ms": prefill16_ms,
            "prefill_B16_tokens_per_s": 16 * 2048 / (prefill16_ms * 1e-3),
            "prefill_B1_T16384_ms": prefill_long_ms,
            "prefill_B1_T16384_tokens_per_s": 16384 / (prefill_long_ms * 1e-3),
            "train_step_B4_T2048_ms": train_ms,
            "train_tokens_per_s": 4 * 2048 / (train_ms * 1e-3),
            "decode_B64_graph_us_per_token": decode_us}


def backward_bench(pkg, wl, torch, reps=3, untimed=2):
    """kda_chunkwise forward + native backward under autograd at the chunkwise
    benchmark shape (fp16 q/k/v, fp32 g/beta, fp32 state from zeros)."""
    inp = wl.make_inputs(B1, T1, H1, D1, D1, device="cuda", seed=1, qkv_dtype=torch.float16)
    xs = [inp[n].clone().requires_grad_(True) for n in ("q", "k", "v", "g", "beta")]
    gen = torch.Generator(device="cuda").manual_seed(3)
    d_o = torch.randn(B1, T1, H1, D1, device="cuda", dtype=torch.float16, generator=gen)
    # `untimed` steps, then `reps` steps queued back to back (no host
    # synchronisation between them, as in a training loop), HIP events around
    # each step's forward and backward on the stream they run on
    for _ in range(untimed):
        for x in xs:
            x.grad = None
        o, _ = pkg.kda_chunkwise(*xs, chunk_size=C1, state_dtype=torch.float32)
        o.backward(d_o)
    torch.cuda.synchronize()
    evs = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(3)) for _ in range(reps)]
    for e0, e1, e2 in evs:
        for x in xs:
            x.grad = None
        e0.record()
        o, _ = pkg.kda_chunkwise(*xs, chunk_size=C1, state_dtype=torch.float32)
        e1.record()
        o.backward(d_o)
        e2.record()
    torch.cuda.synchronize()
    fwd = sum(e0.elapsed_time(e1) for e0, e1, _ in evs) / reps
    bwd = sum(e1.elapsed_time(e2) for _, e1, e2 in evs) / reps
    nbytes = backward_bytes(B1, T1, H1, D1, D1, 2)
    # the gradient's own I/O per (token, head): q, k, v, dO (2 B) and g (4 B) per
    # channel and beta read; dq, dk, dv (2 B), dg (4 B) per channel and dbeta written
    io = B1 * T1 * H1 * (4 * 2 * D1 + 4 * D1 + 4 + 3 * 2 * D1 + 4 * D1 + 4)
    return {"workload": "kda_chunkwise forward (with 32-token checkpoints: state, R, A, L, N) + native backward under "
                        "autograd, B=8 T=4096 H=16 dk=dv=128; fp16 q/k/v, fp32 g/beta",
            "forward_ckpt_ms": fwd, "backward_ms": bwd,
            "train_tokens_per_s": B1 * T1 / ((fwd + bwd) * 1e-3),
            # the gradient I/O over the backward's wall time (autograd's own work
            # included): the backward's roofline fraction as a function
            "gradient_io_bytes": io, "backward_hbm_frac": io / (bwd * 1e-3) / (HBM_PEAK_GBS * 1e9),
            # the bytes this implementation moves (its workspace and the forward's
            # checkpoint records read back included) over the same time
            "backward_bytes": nbytes, "backward_bytes_hbm_frac": nbytes / (bwd * 1e-3) / (HBM_PEAK_GBS * 1e9)}


def backward_bytes(B, T, H, K, V, sz, half_state=True):
    """Algorithmic HBM bytes of kda_chunkwise_bwd's two kernels (activations of
    sz bytes; workspace and checkpoints fp32, except the records' state and R
    and the workspace's dS_end, dP and dR, fp16 with fp16 activations
    (half_state); 32-token chunks): the state kernel completes N in the
    records (reads L_10 and N's two diagonal blocks and block 1's beta, writes
    N_10), reads q, k, g, dO, A, N, beta and writes dS_end, dP, dR; the chunk
    kernel reads the checkpoint (S, R), dS_end, dP, dR, dO, q, k, g, L, N, beta
    (P = N Diag(beta) R is formed in the kernel) and writes dq, dk, dv, dg,
    dbeta."""
    nck = -(-T // 32)
    qk, g, v, beta = B * T * H * K * sz, B * T * H * K * 4, B * T * H * V * sz, B * T * H * 4
    mat = B * H * nck * 32 * 32 * 4
    S = B * H * nck * K * V * (2 if half_state else 4)
    # per 32 x V matrix (R, dP, dR): fp16 with fp16 activations
    RPh = B * H * nck * 32 * V * (2 if half_state else 4)
    nk = 3 * mat // 4 + beta // 2 + mat // 4
    state = 2 * qk + g + v + 2 * mat + beta + S + 2 * RPh
    chunk = 2 * S + 3 * RPh + v + 2 * qk + g + 2 * mat + beta + 2 * qk + v + g + beta
    return nk + state + chunk


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baselines(wl, torch, include_decode=True):
    """The CPU oracle (an op-for-op fp32 restatement of the reference's PyTorch
    algorithm) on the host cores, on bounded samples of the workloads:
    chunkwise B=2 of the B=8 T=4096 H=16 workload (every sequence and head
    costs the same), one warm-up run then the median of three; the long
    context's first 8192 tokens (B=1 H=16, strong decay, initial state), one
    run; 128 chained B=64 decode steps.  Threads: torch's intra-op pool,
    which OMP_NUM_THREADS sizes to this process's CPU share."""
    import math
    from oracle import kda_chunkwise_ref, kda_recurrent_ref
    threads = torch.get_num_threads()
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    bs = 2
    s = wl.make_inputs(bs, T1, H1, D1, D1, device="cpu", seed=1, qkv_dtype=torch.float16)
    runs = []
    for i in range(4):
        t0 = time.perf_counter()
        kda_chunkwise_ref(s["q"], s["k"], s["v"], s["g"], s["beta"], chunk_size=C1,
                          state_dtype=torch.float32)
        if i > 0:
            runs.append(time.perf_counter() - t0)
    tc = sorted(runs)[1]
    del s
    out = {"value": bs * T1 / tc, "unit": "tokens/s", "cores": threads, "kind": "port",
           "sample": f"oracle kda_chunkwise_ref on B={bs} of the B={B1} T={T1} H=16 dk=dv=128 C=64 workload "
                     f"(fp16 inputs upcast to fp32): one warm-up run, then the median of three "
                     f"({', '.join(f'{r:.2f}' for r in runs)} s)",
           "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(), "affinity_cpus": affinity}
    tl = 8192
    s3 = wl.make_inputs(1, tl, H1, D1, D1, device="cpu", seed=3, qkv_dtype=torch.float16,
                        a_log_range=(math.log(4.0), math.log(64.0)), state_std=0.02)
    t0 = time.perf_counter()
    kda_chunkwise_ref(s3["q"], s3["k"], s3["v"], s3["g"], s3["beta"], initial_state=s3["state"], chunk_size=C1,
                      state_dtype=torch.float32)
    t3 = time.perf_counter() - t0
    del s3
    out["long_context_tokens_per_s"] = tl / t3
    out["long_context_sample"] = (f"oracle kda_chunkwise_ref on the first {tl} tokens of the B=1 T=32768 H=16 "
                                  f"long-context workload, one run, {t3:.2f} s")
    if include_decode:
        nst = 128
        d = wl.make_inputs(B2, nst, H2, D1, D1, device="cpu", seed=2, qkv_dtype=torch.float16,
                           gate_dtype=torch.float16, state_std=0.02)
        t0 = time.perf_counter()
        kda_recurrent_ref(d["q"], d["k"], d["v"], d["g"], d["beta"], state=d["state"],
                          state_dtype=torch.float32)
        td = time.perf_counter() - t0
        out["decode_us_per_step"] = td / nst * 1e6
        out["decode_sample"] = (f"oracle kda_recurrent_ref, B=64 H=16 dk=dv=128, {nst} chained "
                                f"steps, {td:.1f} s")
    return out


def load_traffic():
    p = ROOT / "profiles" / "chunkwise_traffic.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get("traffic_bytes_per_launch")
        except (ValueError, OSError):
            return None
    return None


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the KDA core has no multi-GPU path in this "
              "build (heads shard trivially across GPUs; see DESIGN.md). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import __graft_entry__ as ge
    pkg = ge.load_package()
    wl = importlib.import_module("kimi_linear_amd.workloads")
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)

    if args.only == "copy":
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": 1 << 30, "copies": args.steps}), flush=True)
        return

    result = {"metric": METRIC, "unit": "tokens/s", "n_gpus": 1, "higher_is_better": True,
              "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
              "steps": args.steps, "warmup": args.warmup}
    # The headline workload first, on a GPU that has run nothing yet (only
    # the driver's W untimed launches before the K timed ones): the cold-start
    # figure, reported beside the steady-state headline measured at the end.
    cw_inp = chunkwise_inputs(wl, torch) if args.only in (None, "gated", "chunkwise") else None
    cold = None
    if args.only is None:
        wall, launch_ms = chunkwise_bench(pkg, wl, torch, args.steps, args.warmup, cw_inp)
        cold = {"note": "the same K launches measured first in the run, after only W untimed ones, "
                        "while the GPU clock is still ramping up",
                "kernel_ms": launch_ms, "ms_per_step": wall * 1e3 / args.steps,
                "tokens_per_s": B1 * T1 * args.steps / wall}
    if args.only in (None, "decode"):
        if args.decode_variant != "all":
            sets = 5 if args.decode_variant.endswith("rot5") else 1
            us = decode_bench(pkg, wl, torch, sets, in_place=args.decode_variant.startswith("in_place"))
            print(json.dumps({"decode_variant": args.decode_variant, "us_per_step": us}), flush=True)
            return
        us_mall = decode_bench(pkg, wl, torch, 1)
        us_hbm = decode_bench(pkg, wl, torch, 5)
        us_ip = decode_bench(pkg, wl, torch, 1, in_place=True)
        us_ip_hbm = decode_bench(pkg, wl, torch, 5, in_place=True)
        us_copy = copy_bench(torch, 5)
        frac = lambda us: DECODE_BYTES / (us * 1e-6) / 1e9 / HBM_PEAK_GBS  # noqa: E731
        result["decode"] = {
            "workload": "kda_recurrent decode step, B=64 H=16 dk=dv=128, fp32 state, fp16 "
                        "q/k/v/g/beta; 512 chained steps in one hipGraph, 5 state sets stepped in "
                        "turn (320 MiB, more than the 256 MB Infinity Cache holds)",
            "us_per_step": us_hbm,
            "gbs": DECODE_BYTES / (us_hbm * 1e-6) / 1e9,
            "hbm_frac": frac(us_hbm),
            "us_per_step_in_place": us_ip_hbm,
            "hbm_frac_in_place": frac(us_ip_hbm),
            "device_copy_us_rotating_320MiB": us_copy,
            "vs_device_copy": us_copy / us_hbm,
            "cache_resident": {
                "note": "one 64 MiB state set: stays in the Infinity Cache, not an HBM figure",
                "us_per_step": us_mall, "frac_of_hbm_peak": frac(us_mall),
                "us_per_step_in_place": us_ip, "frac_of_hbm_peak_in_place": frac(us_ip)},
        }
        if "value" not in result:
            result.update({"value": us_hbm, "unit": "us/step", "higher_is_better": False,
                           "ms_per_step": us_hbm / 1e3})
    if args.only in (None, "backward"):
        result["backward"] = backward_bench(pkg, wl, torch, reps=max(3, args.steps), untimed=5)
        if "value" not in result:
            result.update({"value": result["backward"]["train_tokens_per_s"], "unit": "tokens/s",
                           "ms_per_step": result["backward"]["forward_ckpt_ms"] + result["backward"]["backward_ms"]})
    if args.only in (None, "long"):
        result["long_context"] = long_context_bench(pkg, wl, torch)
        if "value" not in result:
            result.update({"value": result["long_context"]["tokens_per_s"], "unit": "tokens/s",
                           "ms_per_step": result["long_context"]["ms"]})
    if args.only in (None, "layer"):
        result["layer"] = layer_bench(pkg, torch)
        if "value" not in result:
            result.update({"value": result["layer"]["prefill_tokens_per_s"], "unit": "tokens/s",
                           "ms_per_step": result["layer"]["prefill_B4_T2048_ms"]})
    # The gated leg (the same pipeline with the gate formed in its loads, at
    # least 60 untimed launches) runs right before the headline: under this
    # kind of load the GPU's clock takes ~20 ms to settle (launches run up to
    # 20 % slower meanwhile, measured launch by launch), so the headline's W
    # untimed and K timed launches start on a settled GPU.
    if args.only in (None, "gated"):
        ms = gated_bench(pkg, wl, torch, args.steps, max(args.warmup, 60), cw_inp)
        result["gated"] = {
            "workload": "kda_chunkwise_gated, B=8 T=4096 H=16 dk=dv=128 chunk_size=64; fp16 q/k/v, fp16 gk "
                        "and beta logits, fp32 A_log/dt_bias, fp32 state from zeros",
            "kernel_ms": ms, "tokens_per_s": B1 * T1 / (ms * 1e-3),
            "algorithmic_bytes": GATED_BYTES, "gbs": GATED_BYTES / (ms * 1e-3) / 1e9,
            "hbm_frac": GATED_BYTES / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        if "value" not in result:
            result.update({"value": B1 * T1 / (ms * 1e-3), "unit": "tokens/s", "ms_per_step": ms})
    if args.only in (None, "chunkwise"):
        wall, launch_ms = chunkwise_bench(pkg, wl, torch, args.steps, args.warmup, cw_inp)
        ms_per_step = wall * 1e3 / args.steps
        achieved = CHUNK_BYTES / (launch_ms * 1e-3) / 1e9
        result.update({
            "unit": "tokens/s", "higher_is_better": True,
            "value": B1 * T1 * args.steps / wall,
            "ms_per_step": ms_per_step,
            "config": {"workload": "kda_chunkwise forward, B=8 T=4096 H=16 dk=dv=128 "
                                   "chunk_size=64; fp16 q/k/v, fp32 g/beta, fp32 state from zeros",
                       "global_batch": B1, "seq_len": T1, "heads": H1, "head_dim": D1,
                       "parallelism": "single GPU"},
            "cold_start": cold,
            "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                         "traffic": load_traffic(),
                         "kernel_ms": launch_ms,
                         "mfma_frac_causal": CHUNK_FLOPS / (launch_ms * 1e-3) / 1e12
                         / FP16_PEAK_TFLOPS},
        })
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baselines(wl, torch, include_decode=args.only != "chunkwise")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
