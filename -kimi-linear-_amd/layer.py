"""KDA layer around the native core: the reference's ``KimiDeltaAttention``.

Mirrors ``kimi_linear/kda.py:258-536`` -- same parameters (names and shapes, so a
reference ``state_dict`` loads unchanged), same forward semantics and dispatch
rules -- with the core recurrence running on the gfx950 kernels of
:mod:`kimi_linear_amd.kda`.  The projections are library GEMMs; the
elementwise work between them and the core (short convolutions with their
cache, SiLU, L2 norms, gates; RMSNorm and output gate) runs in the two fused
kernels of :mod:`kimi_linear_amd.layer_ops`.  ``ShortConv``,
``HeadwiseRMSNorm`` and :func:`l2norm` keep the reference's names, parameters
and call signatures, so code that calls them directly (``layer.conv_q(x,
conv_state, use_cache=True)``, ``layer.g_norm(o)``) keeps working; the layer
itself never calls their forwards (it runs the fused kernels).

Under grad mode with parameters or x that require grad, ``forward`` runs the
training path (:meth:`KimiDeltaAttention._train_forward`): the same function,
differentiable end to end -- native backward kernels for the pre-processing
(conv, SiLU, L2 norms, gates) and the output epilogue, the native chunkwise
backward for the core over the whole sequence -- without a cache or state.
Inference runs under ``torch.no_grad()`` or ``torch.inference_mode()``.

Semantics kept from the reference:

* ``_projections`` (``kda.py:399-461``): q, k = l2norm(SiLU(ShortConv(W x)))
  per head, v = SiLU(ShortConv(W_v x)); beta = sigmoid(W_beta x) in fp32;
  g = -exp(A_log) * softplus(W_up W_down x + dt_bias) in fp32.  The gates are
  formed inside the core's loads (``kda_chunkwise_gated`` /
  ``kda_recurrent_gated``) from the gate's up-projection and the beta
  logits, so g and beta are never written to memory.  The T == 1
  cached path updates the conv windows (``kda.py:295-307``); a cached
  multi-token call continues from the cached conv inputs (chunked prefill).
* dispatch (``kda.py:473-536``): ``use_cache`` with T == 1 goes to the
  recurrence; otherwise the chunk size is ``chunk_size`` (or T when
  0 < T < chunk_size), the body runs chunkwise and the remainder through the
  recurrence, chained through the state.
* state dtype (``kda.py:392-396``): an fp32 recurrent state when x is fp16 or
  bf16, else the kernel default (v.dtype).
* ``_output`` (``kda.py:464-470``): head-wise RMSNorm, sigmoid output gate in
  fp32, output projection.  When the whole call is one chunkwise body (T a
  multiple of the chunk size, fp16/bf16 activations, K and V in {64, 128}),
  the norm and the gate can run on the chunk kernel's output tile
  (``kda_chunkwise_fused``: one workgroup per head, the core output never
  written).  ``fuse_output`` chooses: True, False, or None (default) for the
  faster of the two as measured -- fused when B H V / 64 exceeds the 256 CUs
  (265 against 294 us at B=16 T=2048 H=16 d=128), split otherwise (201
  against 250 us at B=4).
"""

from __future__ import annotations

from types import SimpleNamespace

import torch
import torch.nn as nn

from .kda import (KdaError, kda_chunkwise, kda_chunkwise_fused, kda_chunkwise_gated, kda_recurrent,
                  kda_recurrent_gated, long_segments)
from .layer_ops import kda_output, kda_output_train, kda_prep, kda_prep_train


def l2norm(x, eps: float):
    """``kda.py:313-325``: x * min(rsqrt(sum x^2), 1 / eps) over the last
    dimension, reduced in fp32 and returned in x's dtype.  For callers of the
    reference's module-level function; the layer's own L2 norms run inside
    the pre-processing kernel."""
    src = x.dtype
    xf = x.float()
    rstd = (xf * xf).sum(-1, keepdim=True).rsqrt().clamp(max=1.0 / eps)
    return (xf * rstd).to(src)


class HeadwiseRMSNorm(nn.Module):
    """Per-head RMSNorm with a weight ``[H, D]`` (``kda.py:258-279``): the
    reference's ``g_norm`` parameter and forward.  The layer applies the norm
    inside the fused output kernel (:func:`kimi_linear_amd.layer_ops.kda_output`)
    or the chunk kernel's epilogue; this forward serves direct callers."""

    def __init__(self, heads: int, dim: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(heads, dim))
        self.eps = float(eps)

    def forward(self, x):  # x: [B, T, H, D]
        """x * rsqrt(mean over D of x^2 + eps) * weight in fp32, returned in x's dtype."""
        dtype = x.dtype
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (xf * self.weight.float()).to(dtype)


class ShortConv(nn.Module):
    """One causal depthwise convolution (``kda.py:282-310``): an ``nn.Conv1d``
    named ``conv``, so the ``state_dict`` keys (``conv.weight`` ``[D, 1, C]``,
    ``conv.bias``) match the reference's, and its forward for direct callers.
    The layer runs the convolution, with its cache, inside the fused
    pre-processing kernel (:func:`kimi_linear_amd.layer_ops.kda_prep`)."""

    def __init__(self, dim: int, conv_size: int, bias: bool = True):
        super().__init__()
        self.dim = dim
        self.conv_size = conv_size
        self.conv = nn.Conv1d(dim, dim, conv_size, groups=dim, bias=bias)

    def forward(self, x, conv_state=None, use_cache=False):
        """x: [B, T, D].  Without ``use_cache``: the causal convolution (left
        padding of conv_size - 1 zeros), [B, T, D].  With ``use_cache``: x is one
        token [B, 1, D] and ``conv_state`` the last conv_size - 1 inputs
        [B, conv_size - 1, D]; the window sum in fp32 (plus the bias), returned
        in x's dtype with the new state (the window's last conv_size - 1 rows)."""
        if use_cache:
            window = torch.cat([conv_state, x], dim=1)
            w = self.conv.weight.squeeze(1).t().float()            # [C, D]
            out = (window.float() * w).sum(1)
            if self.conv.bias is not None:
                out = out + self.conv.bias.float()
            new_state = window[:, 1 - self.conv_size:] if self.conv_size > 1 else window[:, :0]
            return out.to(x.dtype).unsqueeze(1), new_state
        xt = torch.nn.functional.pad(x.transpose(1, 2), (self.conv_size - 1, 0))
        return self.conv(xt).transpose(1, 2)


def linear_attn_config(**kw) -> SimpleNamespace:
    """A minimal config object with the fields ``KimiDeltaAttention`` reads
    (``kda.py:332-386``); keyword overrides go into ``linear_attn_config``
    except ``hidden_size``, ``l2norm_eps`` and ``rms_norm_eps``."""
    la = dict(num_heads=16, head_dim=128, value_head_dim=128, conv_size=4, chunk_size=64,
              tile_size=0, proj_bias=False, conv_bias=True, gate_low_rank=128,
              output_gate_low_rank=128, a_log_init=0.0, dt_bias_init=0.0)
    top = dict(hidden_size=2048, l2norm_eps=1e-6, rms_norm_eps=1e-6)
    for k, v in kw.items():
        (top if k in top else la)[k] = v
    return SimpleNamespace(linear_attn_config=la, **top)


class KimiDeltaAttention(nn.Module):
    """The KDA layer (``kda.py:331-536``) with the native core."""

    def __init__(self, config):
        super().__init__()
        la = config.linear_attn_config
        d = config.hidden_size
        self.num_heads = la["num_heads"]
        self.head_dim = la["head_dim"]
        self.value_head_dim = la["value_head_dim"]
        self.conv_size = la["conv_size"]
        self.chunk_size = la["chunk_size"]
        self.tile_size = int(la.get("tile_size", 0))
        self.l2norm_eps = config.l2norm_eps
        H, K, V = self.num_heads, self.head_dim, self.value_head_dim
        bias = la["proj_bias"]
        self.in_proj_q = nn.Linear(d, H * K, bias=bias)
        self.in_proj_k = nn.Linear(d, H * K, bias=bias)
        self.in_proj_v = nn.Linear(d, H * V, bias=bias)
        conv_bias = la["conv_bias"]
        self.conv_q = ShortConv(H * K, self.conv_size, bias=conv_bias)
        self.conv_k = ShortConv(H * K, self.conv_size, bias=conv_bias)
        self.conv_v = ShortConv(H * V, self.conv_size, bias=conv_bias)
        self.gk_proj = nn.Sequential(nn.Linear(d, la["gate_low_rank"], bias=bias),
                                     nn.Linear(la["gate_low_rank"], H * K, bias=bias))
        self.A_log = nn.Parameter(torch.zeros(H, K) + float(la["a_log_init"]))
        self.dt_bias = nn.Parameter(torch.zeros(H, K) + float(la["dt_bias_init"]))
        self.beta_proj = nn.Linear(d, H, bias=bias)
        self.og_proj = nn.Sequential(nn.Linear(d, la["output_gate_low_rank"], bias=bias),
                                     nn.Linear(la["output_gate_low_rank"], H * V, bias=bias))
        self.g_norm = HeadwiseRMSNorm(H, V, config.rms_norm_eps)
        self.o_proj = nn.Linear(H * V, d, bias=bias)
        self.fp32_recurrent_state = True
        self._wcat = None          # (key, weight, bias) of the fused input projection
        self._gcat = None          # (key, A_log, dt_bias) in fp32 for the gated core
        self.fuse_output = None    # output epilogue in the chunk kernel: True, False, None = by shape

    def _input_mods(self):
        return (self.in_proj_q, self.in_proj_k, self.in_proj_v, self.beta_proj, self.gk_proj[0], self.og_proj[0])

    def _input_weight(self):
        """The six projections of x -- q, k, v, beta and the down-projections
        of the forget gate and the output gate -- as one ``[N, d]`` weight (and
        bias), so that a step runs one GEMM over x instead of six small ones.

        The module keeps its own parameters (checkpoints load unchanged); the
        concatenation is a cache keyed on every weight's and bias's
        (data_ptr, _version, dtype, device).  Replacing a parameter, or
        updating it in place through autograd-visible ops (``copy_``,
        ``load_state_dict``, an optimizer step), changes the key and refills
        the cache.  A refill of the same shape, dtype and device writes into
        the existing buffers, so a captured decode graph that reads them sees
        the new weights.  Writes through ``.data`` do not bump ``_version``:
        call :meth:`refresh_fused_weight` after them."""
        mods = self._input_mods()
        params = [m.weight for m in mods] + [m.bias for m in mods if m.bias is not None]
        key = tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in params)
        if self._wcat is not None and self._wcat[0] == key:
            return self._wcat[1], self._wcat[2]
        with torch.no_grad():
            w_parts = [m.weight for m in mods]
            b_parts = [m.bias for m in mods] if mods[0].bias is not None else None
            n = sum(p.shape[0] for p in w_parts)
            old = self._wcat
            w0 = w_parts[0]
            if (old is not None and old[1].shape == (n, w0.shape[1]) and old[1].dtype == w0.dtype
                    and old[1].device == w0.device and (old[2] is None) == (b_parts is None)):
                w, b = old[1], old[2]
                torch.cat(w_parts, 0, out=w)
                if b is not None:
                    torch.cat(b_parts, out=b)
            else:
                w = torch.cat(w_parts, 0)
                b = torch.cat(b_parts) if b_parts is not None else None
        self._wcat = (key, w, b)
        return w, b

    def refresh_fused_weight(self) -> None:
        """Refill the concatenated input-projection weight and the fp32 gate
        parameters from the parameters (in place when the layout is
        unchanged).  Needed only after writes that bypass autograd's version
        counter, such as ``p.data.copy_(...)``."""
        if self._wcat is not None:
            self._wcat = (None, self._wcat[1], self._wcat[2])
        if self._gcat is not None:
            self._gcat = (None, self._gcat[1], self._gcat[2])
        self._input_weight()
        self._gate_params()

    def _gate_params(self):
        """``A_log`` and ``dt_bias`` as contiguous fp32 ``[H, K]`` tensors for the
        gated core (the reference casts them to fp32 too, ``kda.py:458-459``);
        cached like :meth:`_input_weight` and refilled in place."""
        params = (self.A_log, self.dt_bias)
        key = tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in params)
        if self._gcat is not None and self._gcat[0] == key:
            return self._gcat[1], self._gcat[2]
        with torch.no_grad():
            old = self._gcat
            if old is not None and old[1].shape == self.A_log.shape and old[1].device == self.A_log.device:
                a, d = old[1], old[2]
                a.copy_(self.A_log)
                d.copy_(self.dt_bias)
            else:
                a = self.A_log.detach().to(torch.float32).clone().contiguous()
                d = self.dt_bias.detach().to(torch.float32).clone().contiguous()
        self._gcat = (key, a, d)
        return a, d

    def _fused_output_ok(self, x):
        if self.fuse_output is False:
            return False
        ok = (x.dtype in (torch.float16, torch.bfloat16) and self.head_dim in (64, 128)
              and self.value_head_dim in (64, 128))
        if self.fuse_output is None:
            # the split kernel runs B H V / 64 workgroups of 64 columns at
            # most; the fused one B H, each somewhat slower: it pays when the
            # split one needs more than one round on the 256 CUs
            ok = ok and x.shape[0] * self.num_heads * (self.value_head_dim // 64) > 256
        return ok

    def _state_dtype(self, x):
        if self.fp32_recurrent_state and x.dtype in (torch.float16, torch.bfloat16):
            return torch.float32
        return None

    def init_state(self, batch: int, device=None, dtype=None) -> dict:
        """An empty decode state (the shape ``forward`` creates for use_cache)."""
        keep = max(self.conv_size - 1, 0)
        H, K, V = self.num_heads, self.head_dim, self.value_head_dim
        z = lambda dim: torch.zeros(batch, keep, dim, device=device, dtype=dtype)  # noqa: E731
        return {"conv": {"q": z(H * K), "k": z(H * K), "v": z(H * V)}, "recurrent": None}

    def _projections(self, x, conv_cache=None, use_cache=False, conv_out=None, gates=False):
        """q, k, v, the gate's up-projection gk ``[B, T, H, K]``, the beta logits
        ``[B, T, H]``, the new conv cache and the output gate's down-projection
        of x (``kda.py:399-461``).

        The projections of x are one library GEMM (:meth:`_input_weight`) and
        the gate's up-projection a second; the three short convolutions with
        their cache, SiLU and the q/k L2 norms are one fused kernel
        (:func:`kda_prep`), and the forget gate and beta are formed by the
        gated core from gk and the logits.  ``gates``: the fused kernel forms
        them instead and g ``[B, T, H, K]``, beta ``[B, T, H]`` (fp32) take the
        places of gk and the logits, for the ungated core.  ``conv_out``: write
        the new conv cache into these tensors (may be ``conv_cache`` itself for
        T <= 16) instead of returning new ones."""
        keep = max(self.conv_size - 1, 0)
        hist = conv_cache if (use_cache and conv_cache is not None and keep > 0) else None
        convs = (self.conv_q.conv, self.conv_k.conv, self.conv_v.conv)
        H, K, V = self.num_heads, self.head_dim, self.value_head_dim
        w, b = self._input_weight()
        y = torch.nn.functional.linear(x, w, b)
        q_in, k_in, v_in, beta_logit, gk_low, og_low = torch.split(
            y, (H * K, H * K, H * V, H, self.gk_proj[0].out_features, self.og_proj[0].out_features), dim=-1)
        gk = self.gk_proj[1](gk_low)
        gate_in = (gk, *self._gate_params(), beta_logit) if gates else (None, None, None, None)
        q, k, v, g, beta, new_conv = kda_prep(
            q_in, k_in, v_in,
            tuple(c.weight for c in convs), tuple(c.bias for c in convs),
            *gate_in,
            num_heads=self.num_heads, head_dim=self.head_dim, value_head_dim=self.value_head_dim,
            l2_eps=self.l2norm_eps, hist=hist, hist_out=conv_out if use_cache else None,
            want_hist=use_cache and conv_out is None)
        if gates:
            return q, k, v, g, beta, new_conv, og_low
        return q, k, v, gk.view(x.shape[0], x.shape[1], H, K), beta_logit, new_conv, og_low

    def _output(self, o_core, og_low):
        """Head-wise RMSNorm, sigmoid output gate (one fused kernel,
        :func:`kda_output`) and the output projection (``kda.py:464-470``);
        ``og_low`` is the output gate's down-projection of x."""
        gate = self.og_proj[1](og_low)
        if gate.dtype != o_core.dtype:
            gate = gate.to(o_core.dtype)
        return self.o_proj(kda_output(o_core, gate, self.g_norm.weight, self.g_norm.eps))

    def decode_step_(self, x, state):
        """One cached decode token (x: [B, 1, d]) that updates ``state`` in
        place and returns out [B, 1, d]: the result of
        ``forward(x, state, use_cache=True)`` with the conv cache and the
        recurrent state ([B, H, K, V], allocated) overwritten by the kernels.  This is the static-state step a captured graph replays;
        the reference instead copies each new state back into its static
        buffers (``graph_decode.py:257-262``), a full extra read and write of
        the state per layer and token."""
        if x.shape[1] != 1:
            raise ValueError(f"decode_step_ takes one token, got x of shape {tuple(x.shape)}")
        q, k, v, gk, bl, _, og_low = self._projections(x, conv_cache=state["conv"], use_cache=True,
                                                       conv_out=state["conv"])
        rec = state["recurrent"]
        if rec is None:
            raise ValueError("decode_step_ needs an allocated recurrent state (run a prefill first)")
        a_log, dt_bias = self._gate_params()
        o_core, _ = kda_recurrent_gated(q, k, v, gk, bl, a_log, dt_bias, state=rec, state_dtype=rec.dtype,
                                        state_out=rec)
        return self._output(o_core, og_low)

    def _train_forward(self, x):
        """The layer's forward for training (``kda.py:473-536`` differentiated by
        autograd in the reference, ``scripts/train_musicgpt_fp16.py:519-523``):
        the six projections of x as one differentiable GEMM over the
        concatenated weights, the pre-processing (:func:`kda_prep_train`: conv,
        SiLU, L2 norms and the gates g, beta), the core over the whole sequence
        (:func:`kda_chunkwise`, any T: the recurrence is chunk-size invariant,
        so the reference's chunkwise body plus recurrent tail is the same
        function), the output epilogue (:func:`kda_output_train`) and o_proj.
        Every step has a native backward; no cache, no state."""
        H, K, V = self.num_heads, self.head_dim, self.value_head_dim
        if K not in (64, 128) or V not in (64, 128):
            # the pre-processing backward (kda_prep_bwd) takes head dims 64 and 128:
            # refuse before any forward work rather than inside backward
            raise KdaError(f"the layer's training path supports head_dim and value_head_dim in (64, 128); got "
                           f"{K} and {V} (run the forward under torch.no_grad())")
        B, T = x.shape[0], x.shape[1]
        mods = self._input_mods()
        w = torch.cat([m.weight for m in mods], 0)
        b = torch.cat([m.bias for m in mods]) if mods[0].bias is not None else None
        y = torch.nn.functional.linear(x, w, b)
        q_in, k_in, v_in, beta_logit, gk_low, og_low = torch.split(
            y, (H * K, H * K, H * V, H, self.gk_proj[0].out_features, self.og_proj[0].out_features), dim=-1)
        if T == 0:
            return self.o_proj(x.new_zeros(B, 0, H * V))
        convs = (self.conv_q.conv, self.conv_k.conv, self.conv_v.conv)
        gk = self.gk_proj[1](gk_low)
        q, k, v, g, beta = kda_prep_train(q_in, k_in, v_in, tuple(c.weight for c in convs),
                                          tuple(c.bias for c in convs), gk, self.A_log, self.dt_bias, beta_logit,
                                          num_heads=H, head_dim=K, value_head_dim=V, l2_eps=self.l2norm_eps)
        C = self.chunk_size if T % self.chunk_size == 0 else T
        o_core, _ = kda_chunkwise(q, k, v, g, beta, chunk_size=C, state_dtype=self._state_dtype(x))
        gate = self.og_proj[1](og_low)
        if gate.dtype != o_core.dtype:
            gate = gate.to(o_core.dtype)
        return self.o_proj(kda_output_train(o_core, gate, self.g_norm.weight, self.g_norm.eps))

    def forward(self, x, state=None, use_cache=False):
        """x: [B, T, d]; ``state`` = {"conv": {"q", "k", "v"}, "recurrent"}.
        Returns out, or (out, new_state) with ``use_cache``.  Under grad mode
        with x or a parameter requiring grad: the training path (no cache, no
        state; see :meth:`_train_forward`)."""
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            if use_cache or state is not None:
                raise KdaError("the training path (grad mode with parameters that require grad) takes no cache "
                               "or state; run cached prefill and decode under torch.no_grad()")
            return self._train_forward(x)
        if use_cache and state is None:
            state = self.init_state(x.shape[0], device=x.device, dtype=x.dtype)
        conv_cache = state["conv"] if state is not None else None
        rec = state["recurrent"] if state is not None else None
        B, T = x.shape[0], x.shape[1]
        sdtype = self._state_dtype(x)
        C = self.chunk_size
        if 0 < T < C:
            C = T
        body = T - T % C if T > 0 else 0
        fused = not (use_cache and T == 1) and T > 0 and T % C == 0 and self._fused_output_ok(x)
        # Few chains over a long body: the ungated core splits the sequence
        # into parallel segments (kda_chunkwise_long_fwd), which the gated one
        # does not, so the pre-processing kernel forms g and beta (B=1 T=4096
        # H=16 d=128: 179 against 347 us for the core).
        split = (not fused and not (use_cache and T == 1) and body > 0 and (B == 1 or body == T)
                 and long_segments(B, body, self.num_heads, self.head_dim, self.value_head_dim, x.dtype) > 1)
        q, k, v, g, beta, new_conv, og_low = self._projections(x, conv_cache=conv_cache, use_cache=use_cache,
                                                               gates=split)
        gate = self._gate_params()      # unless split, g and beta above are gk and the beta logits
        if fused:
            # one chunkwise body and no tail: the output epilogue runs on the
            # chunk kernel's tiles and its result is the o_proj input
            og = self.og_proj[1](og_low)
            y, new_rec = kda_chunkwise_fused(q, k, v, g, beta, *gate, og, self.g_norm.weight, self.g_norm.eps,
                                             initial_state=rec, chunk_size=C, state_dtype=sdtype)
            out = self.o_proj(y)
            if use_cache:
                return out, {"conv": new_conv, "recurrent": new_rec}
            return out
        if use_cache and T == 1:
            o_core, new_rec = kda_recurrent_gated(q, k, v, g, beta, *gate, state=rec, state_dtype=sdtype)
        else:
            rem = T % C
            # every position is written by the body or the tail (the reference
            # zero-fills first, kda.py:516): without a tail the body's output
            # is the result as it is
            o_core = None
            if body > 0 and split:
                o_body, rec = kda_chunkwise(q[:, :body], k[:, :body], v[:, :body], g[:, :body], beta[:, :body],
                                            initial_state=rec, chunk_size=C, state_dtype=sdtype)
            elif body > 0:
                o_body, rec = kda_chunkwise_gated(q[:, :body], k[:, :body], v[:, :body], g[:, :body],
                                                  beta[:, :body], *gate, initial_state=rec, chunk_size=C,
                                                  state_dtype=sdtype)
            if body > 0:
                if rem == 0:
                    o_core = o_body
                else:
                    o_core = x.new_empty(B, T, self.num_heads, self.value_head_dim)
                    o_core[:, :body] = o_body
            if rem > 0 and split:
                o_tail, rec = kda_recurrent(q[:, body:], k[:, body:], v[:, body:], g[:, body:], beta[:, body:],
                                            state=rec, state_dtype=sdtype)
            elif rem > 0:
                o_tail, rec = kda_recurrent_gated(q[:, body:], k[:, body:], v[:, body:], g[:, body:],
                                                  beta[:, body:], *gate, state=rec, state_dtype=sdtype)
            if rem > 0:
                if o_core is None:
                    o_core = o_tail
                else:
                    o_core[:, body:] = o_tail
            if o_core is None:
                o_core = x.new_zeros(B, T, self.num_heads, self.value_head_dim)
            new_rec = rec
        out = self._output(o_core, og_low)
        if use_cache:
            return out, {"conv": new_conv, "recurrent": new_rec}
        return out
