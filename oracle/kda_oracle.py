"""CPU oracle for the Kimi Delta Attention (KDA) core.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path may import, call or
execute this module: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker (or, for
``bench.py``, as the timed CPU baseline).

Two restatements of the reference's algorithms, in fp32 on the CPU:

* :func:`kda_chunkwise_ref` follows ``kimi_linear/kda.py:111-185`` (fp32
  branch): inputs are blocked into chunks of ``chunk_size`` tokens, the
  pairwise decay tensor ``exp(gc_c - gc_i)`` is materialised per chunk
  (``kda.py:159-162``), ``L`` and ``Aout`` are masked reductions over it
  (``kda.py:164-168``), the UT inverse comes from a batched unit-lower
  triangular solve (``kda.py:170-171``) and the chunk loop carries an fp32
  state (``kda.py:172-182``).
* :func:`kda_recurrent_ref` follows ``kda.py:196-219``: the token-by-token
  recurrence with the fp16 output clamp to +-60000 (``kda.py:217-218``,
  ``kimi_linear/fp16.py:97``).

Both keep the reference's signatures and semantics (``kda.py:58-59,188``): q is
scaled by ``K**-0.5`` inside, gates are upcast to fp32, the initial state is
cloned and never mutated, ``o`` has ``v.dtype`` and the state has
``state_dtype or v.dtype``.

:func:`kda_recurrent_f64` is the paper's Eq. 1 (``kda.py:7-10``) written as
explicit matrix products in float64 numpy -- a different formulation of the
same recurrence, used by the tests to pin the fp32 oracle together with the
closed-form special cases in ``tests/test_oracle.py``.

Both compute in fp64 instead when ``v`` is fp64: the tests differentiate them
with autograd (in fp64) as the reference for the native backward.

Pinning status (which independent checks fix each function):
* ``kda_recurrent_ref`` -- fp64 matrix form, closed forms (beta=0 pure decay,
  alpha=1/beta=1 delta-rule write, alpha=0 reset, orthogonal keys), linearity.
* ``kda_chunkwise_ref`` -- equality with the recurrence (a different
  algorithm), chunk-size invariance, split-T chaining, prefix invariance.
* autograd of ``kda_chunkwise_ref`` (the backward reference) -- finite
  differences (``torch.autograd.gradcheck`` in fp64) and equality with
  autograd of ``kda_recurrent_ref``.
No golden vectors ship with the reference for this path (it has no tests), so
no reference-held vector pins either function; see ``tests/test_oracle.py``.
"""

from __future__ import annotations

import numpy as np
import torch

FP16_MAX_SAFE = 60000.0     # kimi_linear/fp16.py:97


def _compute_dtype(x: torch.Tensor) -> torch.dtype:
    """fp32, as the reference computes; fp64 when the caller passes fp64 (the
    tests differentiate the oracle in fp64 to check the native backward)."""
    return torch.float64 if x.dtype == torch.float64 else torch.float32


def _blocks(x: torch.Tensor, B: int, NT: int, C: int, H: int, cd=torch.float32) -> torch.Tensor:
    """[B, T, H, D] -> [B, H, NT, C, D] in fp32 (kda.py:123-127)."""
    return x.to(cd).reshape(B, NT, C, H, x.shape[-1]).permute(0, 3, 1, 2, 4)


def kda_chunkwise_ref(q, k, v, g, beta, initial_state=None, chunk_size=64,
                      tile_size=0, state_dtype=None):
    """fp32 chunkwise KDA forward (restates kimi_linear/kda.py:111-185).

    ``tile_size`` only bounded the reference's transient memory
    (kda.py:101-103); it has no numerical effect and is ignored here.
    """
    del tile_size
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = int(chunk_size)
    if C <= 0 or T % C != 0:
        raise ValueError(f"T={T} must be a multiple of chunk_size={C}")
    NT = T // C
    out_dtype = v.dtype
    cd = _compute_dtype(v)

    Q = _blocks(q, B, NT, C, H, cd) * (K ** -0.5)
    Kb = _blocks(k, B, NT, C, H, cd)
    Vb = _blocks(v, B, NT, C, H, cd)
    G = _blocks(g, B, NT, C, H, cd).cumsum(-2)      # in-chunk cumulative log decay
    Bt = beta.to(cd).reshape(B, NT, C, H).permute(0, 3, 1, 2)

    if initial_state is None:
        S = torch.zeros(B, H, K, V, dtype=cd)
    else:
        S = initial_state.to(cd).clone()
    o = torch.empty(B, H, NT, C, V, dtype=cd)

    eye = torch.eye(C, dtype=cd)
    keep = torch.ones(C, C, dtype=torch.bool).tril()          # i <= c
    strict = torch.ones(C, C, dtype=torch.bool).tril(-1)      # i <  c
    for n in range(NT):
        Qn, Kn, Vn, Gn, bn = Q[:, :, n], Kb[:, :, n], Vb[:, :, n], G[:, :, n], Bt[:, :, n]
        # pairwise decay exp(gc_c - gc_i); pairs above the diagonal are set to
        # -inf before the exp so they contribute exactly zero (kda.py:159-168
        # zeroes them after the reduction instead)
        diff = Gn.unsqueeze(-2) - Gn.unsqueeze(-3)               # [B,H,C(c),C(i),K]
        D = diff.masked_fill(~keep[:, :, None], float("-inf")).exp()
        KD = Kn.unsqueeze(-3) * D                                # k_i * exp(gc_c - gc_i)
        Lm = (Kn.unsqueeze(-2) * KD).sum(-1) * bn.unsqueeze(-1)  # beta_c <k_c, .>
        Lm = Lm.masked_fill(~strict, 0.0)
        Am = (Qn.unsqueeze(-2) * KD).sum(-1)                     # <q~_c, .>, i <= c
        Minv = torch.linalg.solve_triangular(eye + Lm, eye, upper=False,
                                             unitriangular=True)
        M = Minv * bn.unsqueeze(-2)                              # (I+L)^-1 Diag(beta)
        E = Gn.exp()
        W = M @ (E * Kn)
        U = M @ Vn
        P = U - W @ S
        o[:, :, n] = (Qn * E) @ S + Am @ P
        g_last = Gn[..., -1, :]
        S = S * g_last.exp().unsqueeze(-1) \
            + ((g_last.unsqueeze(-2) - Gn).exp() * Kn).transpose(-1, -2) @ P

    o = o.permute(0, 2, 3, 1, 4).reshape(B, T, H, V)
    return o.to(out_dtype), S.to(state_dtype or out_dtype)


def kda_recurrent_ref(q, k, v, g, beta, state=None, state_dtype=None):
    """fp32 token-by-token KDA recurrence (restates kimi_linear/kda.py:196-219)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    out_dtype = v.dtype
    cd = _compute_dtype(v)
    qf = q.to(cd) * (K ** -0.5)
    kf, vf, gf, bf = k.to(cd), v.to(cd), g.to(cd), beta.to(cd)
    S = torch.zeros(B, H, K, V, dtype=cd) if state is None \
        else state.to(cd).clone()
    o = torch.zeros(B, T, H, V, dtype=cd)
    for t in range(T):
        S = S * gf[:, t].exp().unsqueeze(-1)                 # Diag(alpha_t) S
        kt = kf[:, t]
        kS = (kt.unsqueeze(-1) * S).sum(-2)                  # k_t^T S
        bt = bf[:, t].reshape(B, H, 1, 1)
        S = S - bt * kt.unsqueeze(-1) * kS.unsqueeze(-2)
        S = S + bt * kt.unsqueeze(-1) * vf[:, t].unsqueeze(-2)
        o[:, t] = (qf[:, t].unsqueeze(-1) * S).sum(-2)       # S_t^T q~_t
    if out_dtype is torch.float16:
        o = o.clamp(-FP16_MAX_SAFE, FP16_MAX_SAFE)
    return o.to(out_dtype), S.to(state_dtype or out_dtype)


def kda_recurrent_f64(q, k, v, g, beta, state=None):
    """Paper Eq. 1 in float64 matrix form, per (b, h) (kimi_linear/kda.py:7-10):

        S_t = (I - beta_t k_t k_t^T) Diag(exp g_t) S_{t-1} + beta_t k_t v_t^T
        o_t = S_t^T (q_t K^-1/2)

    Returns numpy float64 arrays ``o [B,T,H,V]`` and ``S [B,H,K,V]``.
    """
    qn = np.asarray(q.double() if isinstance(q, torch.Tensor) else q, dtype=np.float64)
    kn = np.asarray(k.double() if isinstance(k, torch.Tensor) else k, dtype=np.float64)
    vn = np.asarray(v.double() if isinstance(v, torch.Tensor) else v, dtype=np.float64)
    gn = np.asarray(g.double() if isinstance(g, torch.Tensor) else g, dtype=np.float64)
    bn = np.asarray(beta.double() if isinstance(beta, torch.Tensor) else beta, dtype=np.float64)
    B, T, H, K = qn.shape
    V = vn.shape[-1]
    S0 = np.zeros((B, H, K, V)) if state is None else np.asarray(
        state.double() if isinstance(state, torch.Tensor) else state, dtype=np.float64)
    o = np.zeros((B, T, H, V))
    S_out = np.zeros((B, H, K, V))
    eye = np.eye(K)
    for b in range(B):
        for h in range(H):
            S = S0[b, h].copy()
            for t in range(T):
                kt = kn[b, t, h][:, None]                       # column vector
                A = (eye - bn[b, t, h] * (kt @ kt.T)) @ np.diag(np.exp(gn[b, t, h]))
                S = A @ S + bn[b, t, h] * (kt @ vn[b, t, h][None, :])
                o[b, t, h] = S.T @ (qn[b, t, h] * K ** -0.5)
            S_out[b, h] = S
    return o, S_out
