"""Pins the backward reference: autograd of the chunkwise oracle.

The reference trains through ``kda_chunkwise`` with autograd
(``kimi_linear/kda.py:58-185``, ``scripts/train_musicgpt_fp16.py:519-523``),
so the gradient of record is the derivative of that function.  The native
backward is checked against autograd of the oracle in fp64; this file checks
that reference itself:

* against central finite differences (``torch.autograd.gradcheck``), for every
  input including the initial state, with a final-state gradient too;
* against autograd of the token recurrence (a different algorithm for the same
  function), on ragged chunk counts and with non-trivial decays.
"""

from __future__ import annotations

import torch

from oracle import kda_chunkwise_ref, kda_recurrent_ref


def _inputs(B, T, H, K, V, seed, state=True):
    gen = torch.Generator().manual_seed(seed)

    def randn(*s):
        return torch.randn(*s, generator=gen, dtype=torch.float64)

    q = torch.nn.functional.normalize(randn(B, T, H, K), dim=-1)
    k = torch.nn.functional.normalize(randn(B, T, H, K), dim=-1)
    v = randn(B, T, H, V)
    g = -torch.nn.functional.softplus(randn(B, T, H, K)) * 0.7
    beta = torch.sigmoid(randn(B, T, H))
    s0 = randn(B, H, K, V) * 0.3 if state else None
    return [q, k, v, g, beta, s0]


def _loss_weights(B, T, H, K, V, seed):
    gen = torch.Generator().manual_seed(seed + 1000)
    return (torch.randn(B, T, H, V, generator=gen, dtype=torch.float64),
            torch.randn(B, H, K, V, generator=gen, dtype=torch.float64))


def test_chunkwise_oracle_gradcheck():
    B, T, H, K, V, C = 1, 8, 1, 4, 3, 4
    xs = [x.requires_grad_(True) for x in _inputs(B, T, H, K, V, seed=1)]

    def f(q, k, v, g, beta, s0):
        o, s = kda_chunkwise_ref(q, k, v, g, beta, initial_state=s0, chunk_size=C,
                                 state_dtype=torch.float64)
        return o, s

    assert torch.autograd.gradcheck(f, xs, eps=1e-6, atol=1e-7, rtol=1e-5)


def test_chunkwise_oracle_grad_matches_recurrence():
    B, T, H, K, V, C = 2, 24, 2, 8, 6, 8
    base = _inputs(B, T, H, K, V, seed=2)
    wo, ws = _loss_weights(B, T, H, K, V, seed=2)
    grads = []
    for use_chunk in (True, False):
        xs = [x.clone().requires_grad_(True) for x in base]
        if use_chunk:
            o, s = kda_chunkwise_ref(*xs[:5], initial_state=xs[5], chunk_size=C, state_dtype=torch.float64)
        else:
            o, s = kda_recurrent_ref(*xs[:5], state=xs[5], state_dtype=torch.float64)
        ((o * wo).sum() + (s * ws).sum()).backward()
        grads.append([x.grad for x in xs])
    for name, a, b in zip(("q", "k", "v", "g", "beta", "s0"), *grads):
        err = ((a - b).norm() / b.norm()).item()
        assert err < 1e-10, (name, err)
