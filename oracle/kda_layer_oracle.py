"""CPU oracle for the KDA layer around the core.

TEST INFRASTRUCTURE ONLY: used by ``tests/`` as the checker of the layer glue in
``kimi_linear_amd.layer``; nothing in the product path imports it.

An fp32 restatement of ``KimiDeltaAttention.forward`` (``kimi_linear/kda.py:473-536``)
with its pieces written out independently of torch's library layers:

* :func:`short_conv_ref` -- the causal depthwise convolution of
  ``kda.py:282-310`` as an explicit sum over the ``conv_size`` taps, with an
  optional history of the last ``conv_size - 1`` inputs (the cached path,
  ``kda.py:295-307``, and chunked prefill, ``kda.py:420-444``);
* :func:`l2norm_ref` -- ``kda.py:313-325``;
* :func:`head_rmsnorm_ref` -- ``kda.py:258-279``;
* :func:`gates_ref` -- the forget gate and beta of ``kda.py:452-460`` (also the
  checker of the gated core entry points);
* :func:`kda_layer_ref` -- projections and gates (``kda.py:399-461``), the
  chunk/tail dispatch (``kda.py:502-530``) over the oracle kernels of
  :mod:`oracle.kda_oracle`, and the output path (``kda.py:464-470``).

Parameters are taken from a ``state_dict`` with the reference's key names.
fp64 inputs stay fp64 (everything else is computed in fp32), and
``keep_graph=True`` keeps the autograd graph to the parameters and x: the
tests differentiate the fp64 oracle to check the layer's training path.

Pinning: ``tests/test_layer_oracle.py`` checks the convolution against
``torch.nn.functional.conv1d``, the norms against ``F.normalize`` and
``F.rms_norm``, and the layer's dispatch and cache handling through
invariances (one-pass prefill == chunked prefill == prefill + token-by-token
decode; chunk size and tail split do not change the result).
"""

from __future__ import annotations

import math

import torch

from .kda_oracle import kda_chunkwise_ref, kda_recurrent_ref


def _f(x):
    """fp64 stays fp64; anything else is computed in fp32."""
    return x if x.dtype == torch.float64 else x.float()


def short_conv_ref(x, weight, bias=None, history=None):
    """Causal depthwise conv.  x: [B, T, D]; weight: [D, 1, C]; history:
    [B, C-1, D] of earlier inputs (zeros when None).  Returns [B, T, D] fp32
    (fp64 for fp64 x)."""
    x = _f(x)
    B, T, D = x.shape
    C = weight.shape[-1]
    w = _f(weight).reshape(D, C)
    if history is None:
        history = torch.zeros(B, C - 1, D, dtype=x.dtype)
    full = torch.cat([_f(history).to(x.dtype), x], dim=1)          # [B, C-1+T, D]
    out = torch.zeros(B, T, D, dtype=x.dtype)
    for c in range(C):
        out = out + full[:, c:c + T] * w[:, c]
    if bias is not None:
        out = out + _f(bias)
    return out


def l2norm_ref(x, eps):
    x = _f(x)
    n = torch.sqrt((x * x).sum(-1, keepdim=True))
    return x / torch.clamp(n, min=eps)


def head_rmsnorm_ref(x, weight, eps):
    x = _f(x)
    return x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps) * _f(weight)


def _linear(x, p, name):
    y = x @ _f(p[name + ".weight"]).t()
    b = p.get(name + ".bias")
    return y + _f(b) if b is not None else y


def _silu(x):
    return x * torch.sigmoid(x)


def _softplus(x):
    return torch.where(x > 20, x, torch.log1p(torch.exp(torch.clamp(x, max=20))))


def gates_ref(gk, beta_logit, a_log, dt_bias):
    """g = -exp(A_log) * softplus(gk + dt_bias) and beta = sigmoid(logit), in fp32
    (``kda.py:452-460``); ``gk: [B, T, H, K]``, ``beta_logit: [B, T, H]``,
    ``a_log, dt_bias: [H, K]``."""
    g = -torch.exp(_f(a_log)) * _softplus(_f(gk) + _f(dt_bias))
    return g, torch.sigmoid(_f(beta_logit))


def kda_layer_ref(params, cfg, x, state=None, use_cache=False, keep_graph=False):
    """fp32 CPU forward of the KDA layer (fp64 for fp64 x and parameters).
    ``cfg`` has ``linear_attn_config``, ``l2norm_eps`` and ``rms_norm_eps`` like
    the reference config.  Returns out, or (out, new_state) with ``use_cache``.
    ``keep_graph``: do not detach params and x (for autograd)."""
    la = cfg.linear_attn_config
    H, K, V, Cs = la["num_heads"], la["head_dim"], la["value_head_dim"], la["conv_size"]
    if keep_graph:
        p = dict(params)
        x = _f(x)
    else:
        p = {k: v.detach().cpu() for k, v in params.items()}
        x = _f(x.detach().cpu())
    cd = x.dtype
    B, T, _ = x.shape
    keep = max(Cs - 1, 0)
    if use_cache and state is None:
        state = {"conv": {"q": torch.zeros(B, keep, H * K, dtype=cd), "k": torch.zeros(B, keep, H * K, dtype=cd),
                          "v": torch.zeros(B, keep, H * V, dtype=cd)}, "recurrent": None}
    conv = state["conv"] if state is not None else None
    rec = state["recurrent"] if state is not None else None

    ins = {"q": _linear(x, p, "in_proj_q"), "k": _linear(x, p, "in_proj_k"), "v": _linear(x, p, "in_proj_v")}
    conv_out, new_conv = {}, None
    hist = use_cache and conv is not None and keep > 0
    for n in ("q", "k", "v"):
        h = _f(conv[n]) if hist else None
        conv_out[n] = short_conv_ref(ins[n], p[f"conv_{n}.conv.weight"], p.get(f"conv_{n}.conv.bias"), h)
    if use_cache:
        new_conv = {}
        for n in ("q", "k", "v"):
            full = torch.cat([_f(conv[n]).to(cd), ins[n]], dim=1) if hist else ins[n]
            new_conv[n] = full[:, full.shape[1] - keep:] if keep else full[:, :0]
    q = l2norm_ref(_silu(conv_out["q"]).view(B, T, H, K), cfg.l2norm_eps)
    k = l2norm_ref(_silu(conv_out["k"]).view(B, T, H, K), cfg.l2norm_eps)
    v = _silu(conv_out["v"]).view(B, T, H, V)
    gk = _linear(_linear(x, p, "gk_proj.0"), p, "gk_proj.1").view(B, T, H, K)
    g, beta = gates_ref(gk, _linear(x, p, "beta_proj"), p["A_log"], p["dt_bias"])

    if use_cache and T == 1:
        o_core, new_rec = kda_recurrent_ref(q, k, v, g, beta, state=rec, state_dtype=torch.float32)
    else:
        C = la["chunk_size"]
        if 0 < T < C:
            C = T
        rem = T % C
        body = T - rem
        sd = torch.float64 if cd == torch.float64 else torch.float32
        parts = []
        if body > 0:
            o_b, rec = kda_chunkwise_ref(q[:, :body], k[:, :body], v[:, :body], g[:, :body],
                                         beta[:, :body], initial_state=rec, chunk_size=C, state_dtype=sd)
            parts.append(o_b)
        if rem > 0:
            o_t, rec = kda_recurrent_ref(q[:, body:], k[:, body:], v[:, body:], g[:, body:],
                                         beta[:, body:], state=rec, state_dtype=sd)
            parts.append(o_t)
        o_core = torch.cat(parts, dim=1) if parts else torch.zeros(B, T, H, V, dtype=cd)
        new_rec = rec
    o = head_rmsnorm_ref(o_core, p["g_norm.weight"], cfg.rms_norm_eps)
    gate = torch.sigmoid(_linear(_linear(x, p, "og_proj.0"), p, "og_proj.1").view(B, T, H, V))
    out = _linear((o * gate).reshape(B, T, H * V), p, "o_proj")
    if use_cache:
        return out, {"conv": new_conv, "recurrent": new_rec}
    return out


def make_layer_params(cfg, seed=0, std=0.02):
    """Random layer parameters with the reference's names and shapes:
    projections N(0, std), conv kernels and biases N(0, std) (conv kernels
    scaled by 10 so the taps matter), A_log ~ U(0, ln 16), dt_bias ~ N(0, 0.1),
    norm weight 1 + N(0, 0.1)."""
    la = cfg.linear_attn_config
    H, K, V, Cs = la["num_heads"], la["head_dim"], la["value_head_dim"], la["conv_size"]
    d = cfg.hidden_size
    gen = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    p = {}

    def lin(name, i, o):
        p[name + ".weight"] = rn(o, i) * std
        if la["proj_bias"]:
            p[name + ".bias"] = rn(o) * std

    lin("in_proj_q", d, H * K)
    lin("in_proj_k", d, H * K)
    lin("in_proj_v", d, H * V)
    for n, dim in (("q", H * K), ("k", H * K), ("v", H * V)):
        p[f"conv_{n}.conv.weight"] = rn(dim, 1, Cs) * std * 10
        if la["conv_bias"]:
            p[f"conv_{n}.conv.bias"] = rn(dim) * std
    lin("gk_proj.0", d, la["gate_low_rank"])
    lin("gk_proj.1", la["gate_low_rank"], H * K)
    p["A_log"] = torch.rand(H, K, generator=gen) * math.log(16.0)
    p["dt_bias"] = rn(H, K) * 0.1
    lin("beta_proj", d, H)
    lin("og_proj.0", d, la["output_gate_low_rank"])
    lin("og_proj.1", la["output_gate_low_rank"], H * V)
    p["g_norm.weight"] = 1.0 + rn(H, V) * 0.1
    lin("o_proj", H * V, d)
    return p
