"""Pins the CPU oracle (oracle/kda_oracle.py) with checks independent of its code.

The reference ships no tests or golden vectors for this path, so the oracle is
pinned by
* the paper's Eq. 1 evaluated in float64 matrix form (a different formulation),
* closed forms of special cases (pure decay, delta-rule write, full reset,
  orthogonal keys) and linearity,
* equality of the two oracle algorithms (UT-transform chunkwise vs the
  token recurrence) plus the reference's own invariance claims:
  chunkwise == recurrent (README.md:160), prefix invariance (README.md:161),
  chunked extension (README.md:187), chunk-size invariance
  (kimi_musicgpt/configs/musicgpt_1p5b.json:6).
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import FP16_MAX_SAFE, kda_chunkwise_ref, kda_recurrent_f64, kda_recurrent_ref


def rand_inputs(B, T, H, K, V, seed=0, a_log_hi=math.log(16.0), state=False):
    gen = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, K, generator=gen), dim=-1)
    k = F.normalize(torch.randn(B, T, H, K, generator=gen), dim=-1)
    v = torch.randn(B, T, H, V, generator=gen)
    a_log = torch.rand(H, K, generator=gen) * a_log_hi
    x = torch.randn(B, T, H, K, generator=gen)
    dt = torch.randn(H, K, generator=gen) * 0.1
    g = -torch.exp(a_log) * F.softplus(x + dt)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    s0 = torch.randn(B, H, K, V, generator=gen) * 0.02 if state else None
    return q, k, v, g, beta, s0


def max_abs(a, b):
    return (a.double() - torch.as_tensor(b).double()).abs().max().item()


def rel(a, b):
    a, b = a.double(), torch.as_tensor(b).double()
    return ((a - b).norm() / b.norm()).item()


# --------------------------------------------------------------------- recurrent
def test_recurrent_matches_f64_matrix_form():
    q, k, v, g, beta, s0 = rand_inputs(2, 24, 3, 8, 6, seed=1, state=True)
    o, s = kda_recurrent_ref(q, k, v, g, beta, state=s0)
    o64, s64 = kda_recurrent_f64(q, k, v, g, beta, state=s0)
    assert max_abs(o, o64) < 1e-6
    assert max_abs(s, s64) < 1e-6


def test_recurrent_beta_zero_is_pure_decay():
    q, k, v, g, _, s0 = rand_inputs(1, 10, 2, 8, 5, seed=2, state=True)
    beta = torch.zeros(1, 10, 2)
    o, s = kda_recurrent_ref(q, k, v, g, beta, state=s0)
    decay = torch.exp(g.double().cumsum(1))                       # [B,T,H,K]
    s_ref = decay[:, -1].unsqueeze(-1) * s0.double()
    assert max_abs(s, s_ref) < 1e-7
    for t in range(10):
        st = decay[:, t].unsqueeze(-1) * s0.double()
        o_ref = (q[:, t].double() / math.sqrt(8)).unsqueeze(-1).mul(st).sum(-2)
        assert max_abs(o[:, t], o_ref) < 1e-7


def test_recurrent_delta_rule_write():
    # alpha = 1, beta = 1, unit keys: after step t the state maps k_t exactly to v_t
    q, k, v, _, _, s0 = rand_inputs(1, 12, 2, 16, 7, seed=3, state=True)
    g = torch.zeros(1, 12, 2, 16)
    beta = torch.ones(1, 12, 2)
    for t in range(1, 13):
        _, s = kda_recurrent_ref(q[:, :t], k[:, :t], v[:, :t], g[:, :t], beta[:, :t], state=s0)
        recalled = (k[:, t - 1].unsqueeze(-1) * s).sum(-2)      # k_t^T S_t
        assert max_abs(recalled, v[:, t - 1]) < 1e-5


def test_recurrent_full_forget():
    # alpha = 0: S_t = beta_t k_t v_t^T and o_t = beta_t (q~_t . k_t) v_t
    q, k, v, _, beta, s0 = rand_inputs(2, 6, 2, 8, 4, seed=4, state=True)
    g = torch.full((2, 6, 2, 8), -1.0e4)
    o, s = kda_recurrent_ref(q, k, v, g, beta, state=s0)
    qk = (q * k).sum(-1) / math.sqrt(8)
    o_ref = (beta * qk).unsqueeze(-1) * v
    s_ref = beta[:, -1].reshape(2, 2, 1, 1) * k[:, -1].unsqueeze(-1) * v[:, -1].unsqueeze(-2)
    assert max_abs(o, o_ref) < 1e-6
    assert max_abs(s, s_ref) < 1e-6


def test_recurrent_orthogonal_keys():
    # alpha = 1, S0 = 0, mutually orthogonal unit keys: writes never interfere
    K, V, T = 8, 5, 8
    gen = torch.Generator().manual_seed(5)
    basis, _ = torch.linalg.qr(torch.randn(K, K, generator=gen))
    k = basis.T.reshape(1, T, 1, K)                               # rows are orthonormal
    q = F.normalize(torch.randn(1, T, 1, K, generator=gen), dim=-1)
    v = torch.randn(1, T, 1, V, generator=gen)
    beta = torch.sigmoid(torch.randn(1, T, 1, generator=gen))
    g = torch.zeros(1, T, 1, K)
    o, s = kda_recurrent_ref(q, k, v, g, beta)
    s_ref = sum(beta[0, t, 0] * torch.outer(k[0, t, 0], v[0, t, 0]) for t in range(T))
    assert max_abs(s[0, 0], s_ref) < 1e-6
    for t in range(T):
        o_ref = sum(beta[0, s_, 0] * (q[0, t, 0] @ k[0, s_, 0]) / math.sqrt(K) * v[0, s_, 0]
                    for s_ in range(t + 1))
        assert max_abs(o[0, t, 0], o_ref) < 1e-6


def test_recurrent_linear_in_v():
    q, k, v1, g, beta, _ = rand_inputs(1, 16, 2, 8, 4, seed=6)
    v2 = torch.randn(v1.shape, generator=torch.Generator().manual_seed(7))
    o1, s1 = kda_recurrent_ref(q, k, v1, g, beta)
    o2, s2 = kda_recurrent_ref(q, k, v2, g, beta)
    o3, s3 = kda_recurrent_ref(q, k, v1 + 2 * v2, g, beta)
    assert max_abs(o3, o1 + 2 * o2) < 1e-5
    assert max_abs(s3, s1 + 2 * s2) < 1e-5


def test_recurrent_fp16_clamp_and_dtypes():
    q, k, v, g, beta, _ = rand_inputs(1, 3, 1, 4, 4, seed=8)
    s0 = torch.full((1, 1, 4, 4), 1.0e6)
    o, s = kda_recurrent_ref(q, k, v.half(), torch.zeros_like(g), beta, state=s0,
                             state_dtype=torch.float32)
    assert o.dtype == torch.float16 and s.dtype == torch.float32
    assert o.abs().max().item() == FP16_MAX_SAFE
    o32, _ = kda_recurrent_ref(q, k, v, torch.zeros_like(g), beta, state=s0)
    assert o32.abs().max().item() > FP16_MAX_SAFE                 # fp32 output is not clamped


def test_recurrent_does_not_mutate_state():
    q, k, v, g, beta, s0 = rand_inputs(1, 5, 2, 8, 4, seed=9, state=True)
    before = s0.clone()
    kda_recurrent_ref(q, k, v, g, beta, state=s0)
    kda_chunkwise_ref(q[:, :4], k[:, :4], v[:, :4], g[:, :4], beta[:, :4], initial_state=s0,
                      chunk_size=4)
    assert torch.equal(s0, before)


# --------------------------------------------------------------------- chunkwise
@pytest.mark.parametrize("a_log_hi,state", [(math.log(16.0), False), (math.log(64.0), True)])
def test_chunkwise_equals_recurrent(a_log_hi, state):
    # configuration 0 shape: B=1, T=256, H=2, dk=dv=64, C=64
    q, k, v, g, beta, s0 = rand_inputs(1, 256, 2, 64, 64, seed=0, a_log_hi=a_log_hi, state=state)
    o_c, s_c = kda_chunkwise_ref(q, k, v, g, beta, initial_state=s0, chunk_size=64)
    o_r, s_r = kda_recurrent_ref(q, k, v, g, beta, state=s0)
    assert max_abs(o_c, o_r) < 2e-6
    assert rel(s_c, s_r) < 2e-6


def test_chunkwise_matches_f64():
    q, k, v, g, beta, s0 = rand_inputs(2, 32, 2, 8, 6, seed=10, state=True)
    o, s = kda_chunkwise_ref(q, k, v, g, beta, initial_state=s0, chunk_size=8)
    o64, s64 = kda_recurrent_f64(q, k, v, g, beta, state=s0)
    assert max_abs(o, o64) < 1e-6
    assert max_abs(s, s64) < 1e-6


def test_chunk_size_invariance():
    q, k, v, g, beta, s0 = rand_inputs(1, 128, 2, 32, 16, seed=11, state=True)
    outs = [kda_chunkwise_ref(q, k, v, g, beta, initial_state=s0, chunk_size=c)
            for c in (16, 32, 64, 128)]
    for o, s in outs[1:]:
        # fp32 rounding of the in-chunk cumulative decay grows with the chunk
        assert max_abs(o, outs[0][0]) < 1e-5
        assert rel(s, outs[0][1]) < 1e-5


def test_chunked_extension():
    # 16 + 32 tokens chained through the state == one 48-token pass (README.md:187)
    q, k, v, g, beta, _ = rand_inputs(1, 48, 2, 16, 8, seed=12)
    o_full, s_full = kda_chunkwise_ref(q, k, v, g, beta, chunk_size=16)
    o_a, s_a = kda_chunkwise_ref(q[:, :16], k[:, :16], v[:, :16], g[:, :16], beta[:, :16],
                                 chunk_size=16)
    o_b, s_b = kda_chunkwise_ref(q[:, 16:], k[:, 16:], v[:, 16:], g[:, 16:], beta[:, 16:],
                                 initial_state=s_a, chunk_size=16)
    assert max_abs(torch.cat([o_a, o_b], 1), o_full) < 1e-6
    assert rel(s_b, s_full) < 1e-6


def test_prefix_invariance():
    q, k, v, g, beta, _ = rand_inputs(1, 64, 2, 16, 8, seed=13)
    o_full, _ = kda_chunkwise_ref(q, k, v, g, beta, chunk_size=16)
    q2, k2, v2 = q.clone(), k.clone(), v.clone()
    q2[:, 32:] = F.normalize(torch.randn(q2[:, 32:].shape), dim=-1)
    v2[:, 32:] = 100.0
    o_pert, _ = kda_chunkwise_ref(q2, k2, v2, g, beta, chunk_size=16)
    assert torch.equal(o_full[:, :32], o_pert[:, :32])


def test_chunkwise_requires_multiple_of_chunk():
    q, k, v, g, beta, _ = rand_inputs(1, 20, 1, 8, 8)
    with pytest.raises(ValueError):
        kda_chunkwise_ref(q, k, v, g, beta, chunk_size=16)
    o, _ = kda_chunkwise_ref(q, k, v, g, beta, chunk_size=20)    # the module's C = T rule
    o_r, _ = kda_recurrent_ref(q, k, v, g, beta)
    assert max_abs(o, o_r) < 1e-6


def test_batch_head_independence():
    q, k, v, g, beta, s0 = rand_inputs(3, 32, 4, 16, 8, seed=14, state=True)
    o, s = kda_chunkwise_ref(q, k, v, g, beta, initial_state=s0, chunk_size=16)
    o1, s1 = kda_chunkwise_ref(q[1:2, :, 2:3], k[1:2, :, 2:3], v[1:2, :, 2:3], g[1:2, :, 2:3],
                               beta[1:2, :, 2:3], initial_state=s0[1:2, 2:3], chunk_size=16)
    assert max_abs(o[1:2, :, 2:3], o1) < 1e-6
    assert max_abs(s[1:2, 2:3], s1) < 1e-6


def test_output_dtypes():
    q, k, v, g, beta, _ = rand_inputs(1, 16, 1, 8, 8)
    o, s = kda_chunkwise_ref(q.half(), k.half(), v.half(), g, beta, chunk_size=16)
    assert o.dtype == torch.float16 and s.dtype == torch.float16
    o, s = kda_chunkwise_ref(q.half(), k.half(), v.half(), g, beta, chunk_size=16,
                             state_dtype=torch.float32)
    assert o.dtype == torch.float16 and s.dtype == torch.float32
