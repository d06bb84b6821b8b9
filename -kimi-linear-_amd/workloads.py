"""Synthetic KDA-core inputs with the distributions of the reference's KDA layer.

The gates follow ``kimi_linear/kda.py:449-460``: q and k are L2-normalised per
head (``l2norm``, q is *not* pre-scaled -- the kernels apply ``K**-0.5``), the
per-channel log decay is ``g = -exp(A_log) * softplus(x + dt_bias)`` and
``beta = sigmoid(.)``.  Draw order (fixed, one generator): q, k, v, A_log, x,
dt_bias, beta-logits, state.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

LN16 = math.log(16.0)


def make_inputs(B: int, T: int, H: int, K: int, V: int, *, device="cpu", seed: int = 0,
                qkv_dtype=torch.float32, gate_dtype=torch.float32,
                a_log_range=(0.0, LN16), state_std: float | None = None,
                state_dtype=torch.float32) -> dict:
    """Return ``dict(q, k, v, g, beta, state)`` drawn on ``device``.

    ``state`` is None unless ``state_std`` is given (then N(0, state_std^2)).
    """
    dev = torch.device(device)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)

    def randn(*shape):
        return torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32)

    q = F.normalize(randn(B, T, H, K), dim=-1)
    k = F.normalize(randn(B, T, H, K), dim=-1)
    v = randn(B, T, H, V)
    lo, hi = a_log_range
    a_log = torch.rand(H, K, generator=gen, device=dev) * (hi - lo) + lo
    x = randn(B, T, H, K)
    dt_bias = randn(H, K) * 0.1
    g = -torch.exp(a_log) * F.softplus(x + dt_bias)
    del x
    beta = torch.sigmoid(randn(B, T, H))
    state = None
    if state_std is not None:
        state = (randn(B, H, K, V) * state_std).to(state_dtype)
    return {
        "q": q.to(qkv_dtype), "k": k.to(qkv_dtype), "v": v.to(qkv_dtype),
        "g": g.to(gate_dtype), "beta": beta.to(gate_dtype), "state": state,
    }


def slice_heads(inp: dict, b: slice, h: slice) -> dict:
    """The (batch, head) sub-problem ``inp[b, :, h]`` -- heads are independent."""
    out = {}
    for name in ("q", "k", "v", "g"):
        out[name] = inp[name][b, :, h]
    out["beta"] = inp["beta"][b, :, h]
    st = inp.get("state")
    out["state"] = None if st is None else st[b, h]
    return out
