"""Fused pre- and post-processing of the KDA layer on gfx950 (C ABI
``kda_prep_fwd`` / ``kda_output_fwd`` in include/kda_hip.h).

* :func:`kda_prep` -- projections to core inputs in one pass: causal short
  convolution + SiLU (+ per-head L2 norm for q and k) of the three
  projections, the forget gate ``g = -exp(A_log) * softplus(gk + dt_bias)``
  and ``beta = sigmoid(beta_logit)`` (``kimi_linear/kda.py:399-461``, with
  ``ShortConv`` ``kda.py:282-310`` and ``l2norm`` ``kda.py:313-325``).
* :func:`kda_output` -- head-wise RMSNorm times the sigmoid output gate
  (``kda.py:258-279, 464-470``), producing the input of ``o_proj``.

HIP tensors only; a missing library or a CPU tensor raises.
"""

from __future__ import annotations

import ctypes

import torch

from . import _native
from .kda import KdaError

_DTYPE_CODE = {torch.float32: _native.DTYPE_F32, torch.float16: _native.DTYPE_F16,
               torch.bfloat16: _native.DTYPE_BF16}
_TILE = 16      # tokens per prep work unit; an in-place conv cache needs T <= this


def _code(name, t):
    if t.dtype not in _DTYPE_CODE:
        raise KdaError(f"{name} must be float32, float16 or bfloat16, got {t.dtype}")
    return _DTYPE_CODE[t.dtype]


def _rows(name, t, shape):
    """A [B, T, D] activation whose channel dimension is contiguous (copied if not)."""
    if tuple(t.shape) != tuple(shape):
        raise KdaError(f"{name} must be {list(shape)}, got {list(t.shape)}")
    if t.stride(-1) != 1:
        t = t.contiguous()
    return t


def _device_check(tensors):
    dev = tensors[0].device
    if dev.type != "cuda" or any(t.device != dev for t in tensors):
        raise KdaError("the fused KDA layer kernels need all tensors on one HIP device "
                       f"(got {', '.join(str(t.device) for t in tensors)}); there is no CPU path")
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        raise KdaError("the fused KDA layer kernels are forward-only: call under torch.no_grad()")
    return dev


def _call(fn, args, dev, what):
    with torch.cuda.device(dev):
        status = fn(ctypes.byref(args), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    if status != _native.STATUS_OK:
        raise KdaError(f"{what} failed: {_native.status_str(status)}")


def kda_prep(q_in, k_in, v_in, conv_w, conv_b, gk, a_log, dt_bias, beta_logit, *, num_heads, head_dim,
             value_head_dim, l2_eps, hist=None, hist_out=None, want_hist=False):
    """Core inputs from the layer's projections.

    ``q_in, k_in: [B, T, H*K]``, ``v_in: [B, T, H*V]``, ``gk: [B, T, H*K]`` (the
    gate's up-projection), ``beta_logit: [B, T, H]``, all in one activation
    dtype; ``conv_w``/``conv_b``: the three ``nn.Conv1d`` weights
    ``[D, 1, conv_size]`` and biases (or None); ``a_log``, ``dt_bias``: ``[H, K]``.
    ``hist``: the conv cache ``{"q", "k", "v"}`` of ``[B, conv_size - 1, D]``
    inputs preceding this call (None = zeros).  ``hist_out``: write the new
    cache into these tensors (they may be ``hist`` itself when ``T <= 16``);
    ``want_hist``: return a new cache instead.

    Returns ``q, k [B, T, H, K]`` and ``v [B, T, H, V]`` in the activation
    dtype, ``g [B, T, H, K]`` and ``beta [B, T, H]`` in fp32, and the new conv
    cache dict (or None).  ``gk=None`` leaves the gates out (``a_log``,
    ``dt_bias`` and ``beta_logit`` are then ignored and g, beta returned as
    None): for a caller that hands gk and the logits to the gated core entry
    points (:func:`kimi_linear_amd.kda.kda_chunkwise_gated`).
    """
    H, K, V = int(num_heads), int(head_dim), int(value_head_dim)
    if q_in.dim() != 3:
        raise KdaError(f"q_in must be [B, T, H*K], got {list(q_in.shape)}")
    B, T = q_in.shape[0], q_in.shape[1]
    Dk, Dv = H * K, H * V
    q_in = _rows("q_in", q_in, (B, T, Dk))
    k_in = _rows("k_in", k_in, (B, T, Dk))
    v_in = _rows("v_in", v_in, (B, T, Dv))
    gates = gk is not None
    if gates:
        gk = _rows("gk", gk, (B, T, Dk))
        beta_logit = _rows("beta_logit", beta_logit, (B, T, H))
    xs = (q_in, k_in, v_in)
    dt = q_in.dtype
    if any(t.dtype != dt for t in (k_in, v_in) + ((gk, beta_logit) if gates else ())):
        raise KdaError("q_in, k_in, v_in, gk and beta_logit must share one dtype")
    cs = conv_w[0].shape[-1]
    keep = cs - 1
    ws = []
    for n, w, D in zip("qkv", conv_w, (Dk, Dk, Dv)):
        if tuple(w.shape) != (D, 1, cs):
            raise KdaError(f"conv_{n} weight must be [{D}, 1, {cs}], got {list(w.shape)}")
        ws.append(w.contiguous())
    wdt = ws[0].dtype
    bs = []
    for n, b, D in zip("qkv", conv_b, (Dk, Dk, Dv)):
        if b is not None:
            if tuple(b.shape) != (D,) or b.dtype != wdt:
                raise KdaError(f"conv_{n} bias must be [{D}] in {wdt}")
            b = b.contiguous()
        bs.append(b)
    if any(w.dtype != wdt for w in ws):
        raise KdaError("the three conv weights must share one dtype")
    if gates:
        a_log = a_log.reshape(-1).contiguous()
        dt_bias = dt_bias.reshape(-1).contiguous()
        if a_log.numel() != Dk or dt_bias.numel() != Dk or a_log.dtype != dt_bias.dtype:
            raise KdaError(f"A_log and dt_bias must be [H, K] = [{H}, {K}] of one dtype")
    hs = [None, None, None]
    if hist is not None:
        for i, (n, D) in enumerate(zip("qkv", (Dk, Dk, Dv))):
            h = hist[n]
            if tuple(h.shape) != (B, keep, D) or h.dtype != dt:
                raise KdaError(f"conv cache {n} must be [{B}, {keep}, {D}] in {dt}, got "
                               f"{list(h.shape)} {h.dtype}")
            hs[i] = h if h.is_contiguous() else h.contiguous()
    if hist_out is not None and want_hist:
        raise KdaError("pass hist_out or want_hist, not both")
    dev = _device_check([*xs, *ws] + ([gk, beta_logit, a_log, dt_bias] if gates else [])
                        + [t for t in bs + hs if t is not None])

    q = torch.empty(B, T, H, K, device=dev, dtype=dt)
    k = torch.empty(B, T, H, K, device=dev, dtype=dt)
    v = torch.empty(B, T, H, V, device=dev, dtype=dt)
    g = torch.empty(B, T, H, K, device=dev, dtype=torch.float32) if gates else None
    beta = torch.empty(B, T, H, device=dev, dtype=torch.float32) if gates else None
    new_hist = None
    if want_hist:
        new_hist = {n: torch.empty(B, keep, D, device=dev, dtype=dt) for n, D in zip("qkv", (Dk, Dk, Dv))}
    elif hist_out is not None:
        for n, D in zip("qkv", (Dk, Dk, Dv)):
            h = hist_out[n]
            if tuple(h.shape) != (B, keep, D) or h.dtype != dt or not h.is_contiguous() or h.device != dev:
                raise KdaError(f"hist_out {n} must be a contiguous [{B}, {keep}, {D}] {dt} tensor on {dev}")
        new_hist = hist_out
    if T == 0:
        if new_hist is not None:
            for i, n in enumerate("qkv"):
                if hs[i] is None:
                    new_hist[n].zero_()
                elif new_hist[n].data_ptr() != hs[i].data_ptr():
                    new_hist[n].copy_(hs[i])
        return q, k, v, g, beta, new_hist

    a = _native.KdaPrepArgs()
    a.B, a.T, a.H, a.K, a.V, a.conv_size = B, T, H, K, V, cs
    for i in range(3):
        a.x[i] = xs[i].data_ptr()
        a.x_stride[i][0], a.x_stride[i][1] = xs[i].stride(0), xs[i].stride(1)
        a.conv_w[i] = ws[i].data_ptr()
        a.conv_b[i] = bs[i].data_ptr() if bs[i] is not None else None
        a.hist_in[i] = hs[i].data_ptr() if hs[i] is not None else None
        a.hist_out[i] = new_hist["qkv"[i]].data_ptr() if new_hist is not None else None
    a.w_dtype = _code("conv weight", ws[0])
    if gates:
        a.gk = gk.data_ptr()
        a.gk_stride[0], a.gk_stride[1] = gk.stride(0), gk.stride(1)
        a.a_log, a.dt_bias = a_log.data_ptr(), dt_bias.data_ptr()
        a.p_dtype = _code("A_log", a_log)
        a.beta_logit = beta_logit.data_ptr()
        a.beta_stride[0], a.beta_stride[1] = beta_logit.stride(0), beta_logit.stride(1)
        a.g, a.beta = g.data_ptr(), beta.data_ptr()
    else:
        a.p_dtype = _native.DTYPE_F32
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.l2_eps = float(l2_eps)
    a.x_dtype = _code("activations", q_in)
    _call(_native.load().kda_prep_fwd, a, dev, f"kda_prep_fwd (B={B}, T={T}, H={H}, K={K}, V={V}, conv {cs})")
    return q, k, v, g, beta, new_hist


def kda_output(o, gate, weight, eps):
    """``o_proj`` input from the core output: ``rmsnorm(o) * weight`` per head,
    rounded to o's dtype, times ``sigmoid(gate)``, rounded again.

    ``o: [B, T, H, V]``, ``gate: [B, T, H*V]`` (same dtype), ``weight: [H, V]``.
    Returns ``[B, T, H*V]``.
    """
    if o.dim() != 4:
        raise KdaError(f"o must be [B, T, H, V], got {list(o.shape)}")
    B, T, H, V = o.shape
    if o.stride(-1) != 1:
        o = o.contiguous()
    gate = _rows("gate", gate, (B, T, H * V))
    if gate.dtype != o.dtype:
        raise KdaError("o and gate must share one dtype")
    if tuple(weight.shape) != (H, V):
        raise KdaError(f"weight must be [{H}, {V}], got {list(weight.shape)}")
    weight = weight.contiguous()
    dev = _device_check([o, gate, weight])
    y = torch.empty(B, T, H * V, device=dev, dtype=o.dtype)
    if y.numel() == 0:
        return y
    a = _native.KdaOutputArgs()
    a.B, a.T, a.H, a.V = B, T, H, V
    a.o = o.data_ptr()
    a.o_stride[0], a.o_stride[1], a.o_stride[2] = o.stride(0), o.stride(1), o.stride(2)
    a.gate = gate.data_ptr()
    a.gate_stride[0], a.gate_stride[1] = gate.stride(0), gate.stride(1)
    a.weight, a.w_dtype = weight.data_ptr(), _code("weight", weight)
    a.y, a.eps, a.x_dtype = y.data_ptr(), float(eps), _code("o", o)
    _call(_native.load().kda_output_fwd, a, dev, f"kda_output_fwd (B={B}, T={T}, H={H}, V={V})")
    return y


def _c(t):
    return t if t.is_contiguous() else t.contiguous()


def kda_prep_backward(q_in, k_in, v_in, conv_w, conv_b, gk, a_log, dt_bias, beta_logit, dq, dk, dv, dg, dbeta, *,
                      num_heads, head_dim, value_head_dim, l2_eps):
    """Gradients of :func:`kda_prep` (a call without a conv cache) from those
    of its outputs: ``dq, dk [B, T, H, K]``, ``dv [B, T, H, V]`` and, with the
    gates, ``dg [B, T, H, K]``, ``dbeta [B, T, H]`` (fp32).

    Returns ``(dq_in, dk_in, dv_in, dw, db, dgk, dbeta_logit, da_log, ddt_bias)``:
    the projections' gradients in their dtype, the conv weights' ``dw`` (three
    ``[D, 1, conv_size]``) and ``db`` (three ``[D]`` or None) in the weights'
    dtype, and for the gates ``dgk [B, T, H*K]``, ``dbeta_logit [B, T, H]``,
    ``da_log``, ``ddt_bias`` (shaped and typed as ``a_log``, ``dt_bias``), or
    None without gates.  Sums over tokens are fp32 and run in a fixed order.
    """
    H, K, V = int(num_heads), int(head_dim), int(value_head_dim)
    B, T = q_in.shape[0], q_in.shape[1]
    Dk, Dv = H * K, H * V
    xs = (_rows("q_in", q_in, (B, T, Dk)), _rows("k_in", k_in, (B, T, Dk)), _rows("v_in", v_in, (B, T, Dv)))
    dt = xs[0].dtype
    dys = tuple(_c(d.to(dt)).view(B, T, D) for d, D in zip((dq, dk, dv), (Dk, Dk, Dv)))
    cs = conv_w[0].shape[-1]
    ws = [_c(w) for w in conv_w]
    wdt = ws[0].dtype
    bs = [_c(b) if b is not None else None for b in conv_b]
    gates = gk is not None
    dev = xs[0].device
    dxs = [torch.empty_like(x, memory_format=torch.contiguous_format) for x in xs]
    dws = [torch.empty(D, cs, device=dev, dtype=torch.float32) for D in (Dk, Dk, Dv)]
    dbs = [torch.empty(D, device=dev, dtype=torch.float32) if b is not None else None
           for b, D in zip(bs, (Dk, Dk, Dv))]
    out_g = (None, None, None, None)
    if gates:
        gk = _rows("gk", gk, (B, T, Dk))
        beta_logit = _rows("beta_logit", beta_logit, (B, T, H))
        al, db_ = _c(a_log.reshape(-1)), _c(dt_bias.reshape(-1))
        dg = _c(dg.float()).view(B, T, Dk)
        dbeta = _c(dbeta.float()).view(B, T, H)
        dgk = torch.empty(B, T, Dk, device=dev, dtype=dt)
        dlogit = torch.empty(B, T, H, device=dev, dtype=dt)
        dal = torch.empty(Dk, device=dev, dtype=torch.float32)
        ddt = torch.empty(Dk, device=dev, dtype=torch.float32)
    if B * T * H > 0:
        lib = _native.load()
        ws_bytes = lib.kda_prep_bwd_workspace_size(B, T, H, K, V, cs)
        work = torch.empty(max(1, (ws_bytes + 3) // 4), device=dev, dtype=torch.float32)
        a = _native.KdaPrepBwdArgs()
        a.B, a.T, a.H, a.K, a.V, a.conv_size = B, T, H, K, V, cs
        for i in range(3):
            a.x[i] = xs[i].data_ptr()
            a.x_stride[i][0], a.x_stride[i][1] = xs[i].stride(0), xs[i].stride(1)
            a.conv_w[i] = ws[i].data_ptr()
            a.conv_b[i] = bs[i].data_ptr() if bs[i] is not None else None
            a.dy[i] = dys[i].data_ptr()
            a.dx[i] = dxs[i].data_ptr()
            a.dw[i] = dws[i].data_ptr()
            a.db[i] = dbs[i].data_ptr() if dbs[i] is not None else None
        a.w_dtype = _code("conv weight", ws[0])
        if gates:
            a.gk = gk.data_ptr()
            a.gk_stride[0], a.gk_stride[1] = gk.stride(0), gk.stride(1)
            a.a_log, a.dt_bias, a.p_dtype = al.data_ptr(), db_.data_ptr(), _code("A_log", al)
            a.beta_logit = beta_logit.data_ptr()
            a.beta_stride[0], a.beta_stride[1] = beta_logit.stride(0), beta_logit.stride(1)
            a.dg, a.dbeta = dg.data_ptr(), dbeta.data_ptr()
            a.dgk, a.dbeta_logit = dgk.data_ptr(), dlogit.data_ptr()
            a.da_log, a.ddt_bias = dal.data_ptr(), ddt.data_ptr()
        else:
            a.p_dtype = _native.DTYPE_F32
        a.l2_eps = float(l2_eps)
        a.x_dtype = _code("activations", xs[0])
        a.workspace = work.data_ptr()
        _call(lib.kda_prep_bwd, a, dev, f"kda_prep_bwd (B={B}, T={T}, H={H}, K={K}, V={V}, conv {cs})")
    else:
        for t in dxs + dws + [d for d in dbs if d is not None] + ([dgk, dlogit, dal, ddt] if gates else []):
            t.zero_()
    if gates:
        out_g = (dgk, dlogit, dal.view_as(a_log).to(a_log.dtype), ddt.view_as(dt_bias).to(dt_bias.dtype))
    dw = tuple(d.view(-1, 1, cs).to(wdt) for d in dws)
    db = tuple(d.to(wdt) if d is not None else None for d in dbs)
    return (dxs[0], dxs[1], dxs[2], dw, db) + out_g


def kda_output_backward(o, gate, weight, eps, dy):
    """Gradients of :func:`kda_output` from ``dy [B, T, H*V]``: ``(do [B, T, H, V],
    dgate [B, T, H*V], dweight [H, V])``, the first two in o's dtype, the
    last in weight's (an fp32 sum over tokens in a fixed order).  The
    rounding of the normalised value counts as the identity."""
    B, T, H, V = o.shape
    if o.stride(-1) != 1:
        o = o.contiguous()
    gate = _rows("gate", gate, (B, T, H * V))
    weight = _c(weight)
    dy = _c(dy.to(o.dtype)).view(B, T, H * V)
    dev = o.device
    do = torch.empty(B, T, H, V, device=dev, dtype=o.dtype)
    dgate = torch.empty(B, T, H * V, device=dev, dtype=o.dtype)
    dw = torch.empty(H * V, device=dev, dtype=torch.float32)
    if do.numel() == 0:
        dw.zero_()
        return do, dgate, dw.view(H, V).to(weight.dtype)
    lib = _native.load()
    work = torch.empty(max(1, (lib.kda_output_bwd_workspace_size(B, T, H, V) + 3) // 4), device=dev,
                       dtype=torch.float32)
    a = _native.KdaOutputBwdArgs()
    a.B, a.T, a.H, a.V = B, T, H, V
    a.o = o.data_ptr()
    a.o_stride[0], a.o_stride[1], a.o_stride[2] = o.stride(0), o.stride(1), o.stride(2)
    a.gate = gate.data_ptr()
    a.gate_stride[0], a.gate_stride[1] = gate.stride(0), gate.stride(1)
    a.weight, a.w_dtype = weight.data_ptr(), _code("weight", weight)
    a.dy, a.d_o, a.dgate, a.dweight = dy.data_ptr(), do.data_ptr(), dgate.data_ptr(), dw.data_ptr()
    a.eps, a.x_dtype, a.workspace = float(eps), _code("o", o), work.data_ptr()
    _call(lib.kda_output_bwd, a, dev, f"kda_output_bwd (B={B}, T={T}, H={H}, V={V})")
    return do, dgate, dw.view(H, V).to(weight.dtype)


class _PrepFn(torch.autograd.Function):
    """kda_prep (with the gates, no conv cache) with the native backward."""

    @staticmethod
    def forward(ctx, q_in, k_in, v_in, wq, wk, wv, bq, bk, bv, gk, beta_logit, a_log, dt_bias, meta):
        H, K, V, eps = meta
        q, k, v, g, beta, _ = kda_prep(q_in, k_in, v_in, (wq, wk, wv), (bq, bk, bv), gk, a_log, dt_bias, beta_logit,
                                       num_heads=H, head_dim=K, value_head_dim=V, l2_eps=eps)
        ctx.save_for_backward(q_in, k_in, v_in, wq, wk, wv, bq, bk, bv, gk, beta_logit, a_log, dt_bias)
        ctx.meta = meta
        return q, k, v, g, beta

    @staticmethod
    def backward(ctx, dq, dk, dv, dg, dbeta):
        q_in, k_in, v_in, wq, wk, wv, bq, bk, bv, gk, beta_logit, a_log, dt_bias = ctx.saved_tensors
        H, K, V, eps = ctx.meta
        B, T = q_in.shape[0], q_in.shape[1]
        z = lambda *s: torch.zeros(*s, device=q_in.device, dtype=torch.float32)  # noqa: E731
        dq = dq if dq is not None else z(B, T, H, K)
        dk = dk if dk is not None else z(B, T, H, K)
        dv = dv if dv is not None else z(B, T, H, V)
        dg = dg if dg is not None else z(B, T, H, K)
        dbeta = dbeta if dbeta is not None else z(B, T, H)
        dqi, dki, dvi, dw, db, dgk, dlogit, dal, ddt = kda_prep_backward(
            q_in, k_in, v_in, (wq, wk, wv), (bq, bk, bv), gk, a_log, dt_bias, beta_logit, dq, dk, dv, dg, dbeta,
            num_heads=H, head_dim=K, value_head_dim=V, l2_eps=eps)
        return (dqi, dki, dvi, dw[0], dw[1], dw[2], db[0], db[1], db[2], dgk, dlogit, dal, ddt, None)


class _OutputFn(torch.autograd.Function):
    """kda_output with the native backward."""

    @staticmethod
    def forward(ctx, o, gate, weight, eps):
        ctx.save_for_backward(o, gate, weight)
        ctx.eps = eps
        return kda_output(o, gate, weight, eps)

    @staticmethod
    def backward(ctx, dy):
        o, gate, weight = ctx.saved_tensors
        do, dgate, dw = kda_output_backward(o, gate, weight, ctx.eps, dy)
        return do, dgate, dw, None


def kda_prep_train(q_in, k_in, v_in, conv_w, conv_b, gk, a_log, dt_bias, beta_logit, *, num_heads, head_dim,
                   value_head_dim, l2_eps):
    """:func:`kda_prep` with the gates and without a conv cache, differentiable
    (native forward and backward kernels): ``(q, k, v, g, beta)``."""
    return _PrepFn.apply(q_in, k_in, v_in, *conv_w, *conv_b, gk, beta_logit, a_log, dt_bias,
                         (int(num_heads), int(head_dim), int(value_head_dim), float(l2_eps)))


def kda_output_train(o, gate, weight, eps):
    """:func:`kda_output`, differentiable (native forward and backward kernels)."""
    return _OutputFn.apply(o, gate, weight, float(eps))
