"""Drop-in ``kda_chunkwise`` / ``kda_recurrent`` backed by the gfx950 HIP kernels.

Same signatures and semantics as the reference kernels
(``kimi_linear/kda.py:58-59`` and ``kimi_linear/kda.py:188``):

* ``q, k: [B, T, H, K]``, ``v: [B, T, H, V]``, ``g: [B, T, H, K]`` (log decay),
  ``beta: [B, T, H]``; the optional state is ``[B, H, K, V]``.
* q is scaled by ``K**-0.5`` inside (``kda.py:132,141,199``).
* Gates and the state may come in any of fp32 / fp16 / bf16; they are read in
  that dtype and computed in fp32.
* Inputs are never modified; ``o`` is a new ``[B, T, H, V]`` tensor in
  ``v.dtype`` and the state a new ``[B, H, K, V]`` tensor in
  ``state_dtype or v.dtype`` (``kda.py:185,219``).  The one opt-in exception
  is ``kda_recurrent(..., state_out=state)``, an in-place state update.
* ``kda_recurrent`` clamps an fp16 ``o`` to +-60000 (``kda.py:217-218``);
  ``kda_chunkwise`` does not.
* ``kda_chunkwise`` requires ``T % chunk_size == 0`` (``kda.py:109``); the
  reference fails in ``reshape`` with a RuntimeError, this wrapper raises
  :class:`KdaError`, which is both a ValueError and a RuntimeError.
  ``chunk_size`` has no other effect (the maths is chunk-size invariant) and
  ``tile_size`` is accepted and ignored (a memory knob, ``kda.py:101-103``).

Differences that are deliberate:

* HIP tensors only.  There is no CPU path and no fallback: CPU tensors, a
  missing ``libkda_hip.so`` or an unsupported head size raise.
* ``kda_chunkwise`` and ``kda_recurrent`` are differentiable: under grad
  mode, with any input that requires grad, each runs as a
  ``torch.autograd.Function`` whose backward is the native kernel
  ``kda_chunkwise_bwd`` (the reference is differentiated by autograd through
  its torch ops).  The recurrence and the chunkwise form are one function of
  the inputs, so the recurrence's backward recomputes the chunkwise forward's
  checkpoints and runs the same kernels, with the fp16 output clamp's mask
  applied to the incoming gradient.  Head dims K in {32, 64, 128} and V a
  multiple of 32.

Every call is asynchronous on the current stream, allocates only through the
torch caching allocator and never synchronises, so it can be captured in a
``torch.cuda.CUDAGraph`` (the reference captures ``kda_recurrent`` at
``kimi_linear/graph_decode.py:285-287``).
"""

from __future__ import annotations

import ctypes

import torch

from . import _native

FP16_MAX_SAFE = 60000.0     # kimi_linear/fp16.py:97

_DTYPE_CODE = {
    torch.float32: _native.DTYPE_F32,
    torch.float16: _native.DTYPE_F16,
    torch.bfloat16: _native.DTYPE_BF16,
}


class KdaError(ValueError, RuntimeError):
    """Invalid arguments or a failed native call."""


def _check_tensor(name, x):
    if not isinstance(x, torch.Tensor):
        raise KdaError(f"{name} must be a torch.Tensor, got {type(x).__name__}")


def _as_kernel_input(x: torch.Tensor) -> torch.Tensor:
    """A [B, T, H, D] view whose last dimension is contiguous and whose token
    rows do not overlap (stride(1) >= D), copying only if it is not."""
    if x.shape[-1] > 1 and x.stride(-1) != 1:
        return x.contiguous()
    if x.shape[1] > 1 and x.stride(1) < x.shape[-1]:
        return x.contiguous()
    return x


def _beta_input(x: torch.Tensor) -> torch.Tensor:
    """A [B, T, H] view with distinct token rows (stride(1) >= 1)."""
    if x.shape[1] > 1 and x.stride(1) < 1:
        return x.contiguous()
    return x


def _float_or_f32(x: torch.Tensor) -> torch.Tensor:
    return x if x.dtype in _DTYPE_CODE else x.float()


def _strides3(x: torch.Tensor):
    return (ctypes.c_int64 * 3)(*x.stride()[:3])


def _forward(kind, q, k, v, g, beta, state, chunk_size, state_dtype, state_out=None, ckpt=False, gate=None,
             epilogue=None):
    """Shared forward.  ``ckpt=True`` (chunkwise, inside the autograd
    function) also returns the fp32 state before every 32-token chunk.
    ``gate=(a_log, dt_bias)``: g and beta are the gate's up-projection gk
    and the beta logits, and the kernels form the gates (the gated entry
    points).  ``epilogue=(og, weight, eps)`` (chunkwise): the output is the
    layer's o_proj input y instead of o (kda_chunkwise_fused_fwd)."""
    for name, x in (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta)):
        _check_tensor(name, x)
    if state is not None:
        _check_tensor("state", state)
    if state_out is not None:
        _check_tensor("state_out", state_out)
    if q.dim() != 4 or v.dim() != 4:
        raise KdaError(f"q and v must be [B, T, H, D]; got q {tuple(q.shape)}, v {tuple(v.shape)}")
    B, T, H, K = q.shape
    V = v.shape[-1]
    if tuple(k.shape) != (B, T, H, K) or tuple(g.shape) != (B, T, H, K):
        raise KdaError(f"k and g must match q's shape {tuple(q.shape)}; "
                       f"got k {tuple(k.shape)}, g {tuple(g.shape)}")
    if tuple(v.shape[:3]) != (B, T, H):
        raise KdaError(f"v must be [B, T, H, V] = [{B}, {T}, {H}, V]; got {tuple(v.shape)}")
    if tuple(beta.shape) != (B, T, H):
        raise KdaError(f"beta must be [B, T, H] = [{B}, {T}, {H}]; got {tuple(beta.shape)}")
    if state is not None and tuple(state.shape) != (B, H, K, V):
        raise KdaError(f"state must be [B, H, K, V] = [{B}, {H}, {K}, {V}]; got {tuple(state.shape)}")
    if kind == "chunkwise":
        if chunk_size <= 0:
            raise KdaError(f"chunk_size must be positive, got {chunk_size}")
        if T % chunk_size != 0:
            raise KdaError(f"T={T} must be a multiple of chunk_size={chunk_size} "
                           "(the caller splits the body and the tail)")
    if K <= 0 or V <= 0:
        raise KdaError(f"head dims must be positive, got K={K}, V={V}")

    if gate is not None:
        for name, x in zip(("a_log", "dt_bias"), gate):
            _check_tensor(name, x)
            if x.numel() != H * K:
                raise KdaError(f"{name} must be [H, K] = [{H}, {K}]; got {tuple(x.shape)}")

    dev = q.device
    tensors = [q, k, v, g, beta] + [x for x in (state, state_out) if x is not None] + list(gate or ())
    if dev.type != "cuda" or any(x.device != dev for x in tensors):
        raise KdaError("the HIP KDA kernels need all inputs on one HIP device "
                       f"(got {', '.join(str(x.device) for x in tensors)}); there is no CPU path")
    if torch.is_grad_enabled() and any(x.requires_grad for x in tensors):
        raise KdaError("the HIP KDA kernels are forward-only: call under torch.no_grad() "
                       "or detach the inputs")
    if v.dtype not in _DTYPE_CODE:
        raise KdaError(f"v must be float32, float16 or bfloat16, got {v.dtype}")

    out_dtype = v.dtype
    s_dtype = state_dtype or out_dtype
    if not isinstance(s_dtype, torch.dtype) or not s_dtype.is_floating_point:
        raise KdaError(f"state_dtype must be a floating dtype, got {state_dtype!r}")
    kernel_s_dtype = s_dtype if s_dtype in _DTYPE_CODE else torch.float32
    if state_out is not None:
        if tuple(state_out.shape) != (B, H, K, V) or not state_out.is_contiguous():
            raise KdaError(f"state_out must be a contiguous [B, H, K, V] = [{B}, {H}, {K}, {V}] tensor; "
                           f"got {tuple(state_out.shape)} with strides {state_out.stride()}")
        if state_out.dtype != s_dtype or s_dtype not in _DTYPE_CODE:
            raise KdaError(f"state_out must have the state dtype {s_dtype} (float32, float16 or bfloat16); "
                           f"got {state_out.dtype}")
        if state_out.requires_grad and torch.is_grad_enabled():
            raise KdaError("state_out is written in place: it must not require grad under grad mode")

    if epilogue is not None:
        og, w_norm, eps = epilogue
        _check_tensor("og", og)
        _check_tensor("norm weight", w_norm)
        if tuple(og.shape) != (B, T, H * V) or og.device != dev:
            raise KdaError(f"og must be [B, T, H*V] = [{B}, {T}, {H * V}] on {dev}; got {tuple(og.shape)}")
        if w_norm.numel() != H * V:
            raise KdaError(f"the norm weight must be [H, V] = [{H}, {V}]; got {tuple(w_norm.shape)}")
        if v.dtype not in (torch.float16, torch.bfloat16) or K not in (64, 128) or V not in (64, 128):
            raise KdaError("the fused output epilogue takes fp16 / bf16 q, k, v and K, V in (64, 128)")
        og = og.to(v.dtype)
        if og.stride(-1) != 1 or (T > 1 and og.stride(1) < H * V):
            og = og.contiguous()
        epilogue = (og, w_norm.detach().reshape(H, V).to(torch.float32).contiguous(), float(eps))
    o = torch.empty(B, T, H, V, device=dev, dtype=out_dtype)
    s_out = state_out if state_out is not None else torch.empty(B, H, K, V, device=dev, dtype=kernel_s_dtype)
    # per 32-token chunk a record: the state before it (K rows) and the chunk's R
    # (32 rows), all V wide, then its A, L and N (32 x 32 each)
    ck = torch.empty(B, H, (T + CKPT_SPACING - 1) // CKPT_SPACING, ckpt_record(K, V), device=dev,
                     dtype=torch.float32) if ckpt else None
    if B * H == 0:
        if state is not None:
            s_out.copy_(state)
        return (o, s_out.to(s_dtype), ck) if ckpt else (o, s_out.to(s_dtype))

    qk_dtype = out_dtype
    q = _as_kernel_input(q if q.dtype == qk_dtype else q.to(qk_dtype))
    k = _as_kernel_input(k if k.dtype == qk_dtype else k.to(qk_dtype))
    v = _as_kernel_input(v)
    if gate is not None:
        if kind == "chunkwise" and qk_dtype != torch.float32:
            # the chunk pipeline reads gk and the logits in the dtype of q, k and v
            g, beta = g.to(qk_dtype), beta.to(qk_dtype)
        gate = tuple(x.detach().reshape(H, K).to(torch.float32).contiguous() for x in gate)
    elif kind == "chunkwise":
        # the chunkwise pipeline reads fp32 gates (the reference upcasts them too, kda.py:119-120)
        g = g.float()
        beta = beta.float()
    g = _as_kernel_input(_float_or_f32(g))
    beta = _beta_input(_float_or_f32(beta))
    if state is not None:
        state = _float_or_f32(state)
        if not state.is_contiguous():
            state = state.contiguous()
        if state_out is not None and state.data_ptr() != s_out.data_ptr():
            # the kernel reads a state slice before writing it: only an exact
            # alias (in-place update) or disjoint memory is allowed
            n_in = state.numel() * state.element_size()
            n_out = s_out.numel() * s_out.element_size()
            if state.data_ptr() < s_out.data_ptr() + n_out and s_out.data_ptr() < state.data_ptr() + n_in:
                raise KdaError("state_out partially overlaps state: pass the same tensor (in place) "
                               "or disjoint memory")

    args = _native.KdaFwdArgs()
    args.B, args.T, args.H, args.K, args.V = B, T, H, K, V
    args.q, args.k, args.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    args.g, args.beta = g.data_ptr(), beta.data_ptr()
    args.q_stride, args.k_stride, args.v_stride = _strides3(q), _strides3(k), _strides3(v)
    args.g_stride, args.beta_stride = _strides3(g), _strides3(beta)
    args.qkv_dtype = _DTYPE_CODE[qk_dtype]
    args.g_dtype = _DTYPE_CODE[g.dtype]
    args.beta_dtype = _DTYPE_CODE[beta.dtype]
    args.state_in = state.data_ptr() if state is not None else None
    args.state_in_dtype = _DTYPE_CODE[state.dtype] if state is not None else _native.DTYPE_F32
    args.state_out = s_out.data_ptr()
    args.state_out_dtype = _DTYPE_CODE[kernel_s_dtype]
    args.o = o.data_ptr()
    args.scale = float(K) ** -0.5
    args.clamp_fp16_out = 1 if kind == "recurrent" else 0
    args.chunk_size = chunk_size if kind == "chunkwise" else 1

    lib = _native.load()
    with torch.cuda.device(dev):
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        segments = 1
        if kind == "chunkwise" and not ckpt and gate is None and epilogue is None and state_out is None:
            # one batch stride must serve the split views (sequences back to back)
            if B == 1 or all(x.stride(0) == T * x.stride(1) for x in (q, k, v, g, beta)):
                segments = long_segments(B, T, H, K, V, qk_dtype)
        if segments > 1:
            ws = torch.empty(int(lib.kda_chunkwise_long_workspace_size(B, T, H, K, V, segments)), device=dev,
                             dtype=torch.uint8)
            status = lib.kda_chunkwise_long_fwd(ctypes.byref(args), ctypes.c_int64(segments),
                                                ctypes.c_void_p(ws.data_ptr()), stream)
        elif epilogue is not None:
            gargs = None
            if gate is not None:
                gargs = _native.KdaGateArgs()
                gargs.a_log, gargs.dt_bias = gate[0].data_ptr(), gate[1].data_ptr()
            eargs = _native.KdaOutEpilogue()
            eargs.gate = epilogue[0].data_ptr()
            eargs.gate_stride[0], eargs.gate_stride[1] = epilogue[0].stride(0), epilogue[0].stride(1)
            eargs.weight, eargs.eps = epilogue[1].data_ptr(), epilogue[2]
            status = lib.kda_chunkwise_fused_fwd(ctypes.byref(args), ctypes.byref(gargs) if gargs else None,
                                                 ctypes.byref(eargs), stream)
        elif gate is not None:
            gargs = _native.KdaGateArgs()
            gargs.a_log, gargs.dt_bias = gate[0].data_ptr(), gate[1].data_ptr()
            fn = lib.kda_chunkwise_gated_fwd if kind == "chunkwise" else lib.kda_recurrent_gated_fwd
            status = fn(ctypes.byref(args), ctypes.byref(gargs), stream)
        elif ckpt:
            status = lib.kda_chunkwise_fwd_ckpt(ctypes.byref(args), ctypes.c_void_p(ck.data_ptr()), stream)
        elif kind == "chunkwise":
            status = lib.kda_chunkwise_fwd(ctypes.byref(args), stream)
        else:
            status = lib.kda_recurrent_fwd(ctypes.byref(args), stream)
    if status != _native.STATUS_OK:
        name = "fused" if epilogue is not None else ("gated" if gate is not None else "")
        raise KdaError(f"kda_{kind}{'_' + name if name else ''}_fwd failed: {_native.status_str(status)} "
                       f"(B={B}, T={T}, H={H}, K={K}, V={V})")
    if kernel_s_dtype != s_dtype:
        s_out = s_out.to(s_dtype)
    return (o, s_out, ck) if ckpt else (o, s_out)


CKPT_SPACING = 32   # tokens between the forward's state checkpoints (kda_chunkwise_fwd_ckpt)


def ckpt_record(K: int, V: int) -> int:
    """Floats of one chunk's record in kda_chunkwise_fwd_ckpt's output."""
    return (K + CKPT_SPACING) * V + 3 * CKPT_SPACING * CKPT_SPACING
LONG_MIN_SEGMENT = 1024    # shortest segment worth the three-pass split (kda_chunkwise_long_fwd)
FEW_CHAIN_MIN_SEGMENT = 256   # shortest segment of the few-chain form
CU_COUNT = 256


def long_segments(B, T, H, K, V, dtype) -> int:
    """Segments for kda_chunkwise_long_fwd; 1 (one pass) when the chains alone
    fill half the CUs or the shape has no split kernel.

    With V + K a multiple of 128 and V <= 256 the split takes its few-chain
    form whenever its first pass (every segment's state columns and transition
    columns, 128-column workgroups) fits one round of workgroups: the first
    pass then also keeps the outputs from a zero state and their initial-state
    coefficients, and a short pass adds the coefficients times the composed
    initial states.  So P is the largest power of two with B P H (V + K) / 128
    <= the CUs and segments of at least FEW_CHAIN_MIN_SEGMENT tokens.
    Measured (fp16, H=16, d=128, us): B=1 T=32768 543 with 8 segments (600
    with 16 in three passes), B=1 T=16384 301 (331), B=1 T=4096 95 with 8
    (293 in one pass), B=2 T=2048 84 with 4 (150), B=3 T=2048 138 with 2
    (150); B=4 T=2048 161 with 2 against 156 in one pass (the chains fill
    half the CUs: one pass).

    Otherwise the three-pass form: the largest power of two that keeps the
    third pass (every segment's chain from its true initial state) within one
    round of workgroups -- 128-column workgroups when V is a multiple of 128,
    else 64-column ones -- and segments of at least LONG_MIN_SEGMENT tokens,
    and 1 when fewer than 4 segments would result (with 2 the split is slower
    than one pass)."""
    if dtype not in (torch.float16, torch.bfloat16) or K not in (64, 128) or V % 64 != 0:
        return 1
    tiles = B * H * (V // 64)
    if tiles == 0 or 2 * tiles >= CU_COUNT:
        return 1
    P = 1
    if (V + K) % 128 == 0 and V <= 256:
        units = B * H * ((V + K) // 128)
        while (2 * P * units <= CU_COUNT and T % (2 * P) == 0 and T // (2 * P) >= FEW_CHAIN_MIN_SEGMENT):
            P *= 2
        return P
    units = B * H * (V // 128) if V % 128 == 0 else tiles
    while (2 * P * units <= CU_COUNT and T % (2 * P) == 0 and T // (2 * P) >= LONG_MIN_SEGMENT):
        P *= 2
    return P if P >= 4 else 1
BWD_TILE = 32       # the native backward takes V in multiples of this


def _f32c(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.float32).contiguous()


def _chunkwise_backward(q, k, v, g, beta, ckpt, d_o, d_state, need_d_state_in):
    """dq, dk, dv (in v's dtype), dg, dbeta (fp32) and dS_0 from the native backward.

    q, k and v share v's dtype (the forward read them so); the kernels read
    them, and ``d_o`` in the same dtype, as they are and write dq, dk, dv in it."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    dev = q.device
    io = v.dtype if v.dtype in _DTYPE_CODE else torch.float32
    q, k, v = (x.to(io).contiguous() for x in (q, k, v))
    d_o = d_o.to(io).contiguous()
    g, beta = _f32c(g), _f32c(beta)
    d_state = _f32c(d_state) if d_state is not None else None
    dq = torch.empty(B, T, H, K, device=dev, dtype=io)
    dk = torch.empty_like(dq)
    dv = torch.empty(B, T, H, V, device=dev, dtype=io)
    dg = torch.empty(B, T, H, K, device=dev, dtype=torch.float32)
    dbeta = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    ds0 = torch.empty(B, H, K, V, device=dev, dtype=torch.float32) if need_d_state_in else None
    lib = _native.load()
    ws = torch.empty(max(int(lib.kda_chunkwise_bwd_workspace_size(B, T, H, K, V)), 1),
                     device=dev, dtype=torch.uint8)
    args = _native.KdaBwdArgs()
    args.B, args.T, args.H, args.K, args.V = B, T, H, K, V
    args.q, args.k, args.v, args.g, args.beta = (x.data_ptr() for x in (q, k, v, g, beta))
    args.ckpt, args.d_o = ckpt.data_ptr(), d_o.data_ptr()
    args.d_state_out = d_state.data_ptr() if d_state is not None else None
    args.dq, args.dk, args.dg = dq.data_ptr(), dk.data_ptr(), dg.data_ptr()
    args.dbeta, args.dv = dbeta.data_ptr(), dv.data_ptr()
    args.d_state_in = ds0.data_ptr() if ds0 is not None else None
    args.workspace = ws.data_ptr()
    args.scale = float(K) ** -0.5
    args.io_dtype = _DTYPE_CODE[io]
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        status = lib.kda_chunkwise_bwd(ctypes.byref(args), ctypes.c_void_p(stream))
    if status != _native.STATUS_OK:
        raise KdaError(f"kda_chunkwise_bwd failed: {_native.status_str(status)} "
                       f"(B={B}, T={T}, H={H}, K={K}, V={V})")
    return dq, dk, dv, dg, dbeta, ds0


class _ChunkwiseFn(torch.autograd.Function):
    """kda_chunkwise with the native backward (state checkpoints every 32 tokens)."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, initial_state, chunk_size, state_dtype):
        o, s, ckpt = _forward("chunkwise", q, k, v, g, beta, initial_state, chunk_size, state_dtype, ckpt=True)
        # the kernel read q and k in v's dtype and the gates in fp32: differentiate that function
        ctx.save_for_backward(q.to(v.dtype), k.to(v.dtype), v, g.float(), beta.float(), ckpt)
        ctx.dtypes = (q.dtype, k.dtype, v.dtype, g.dtype, beta.dtype,
                      initial_state.dtype if initial_state is not None else None)
        return o, s

    @staticmethod
    def backward(ctx, d_o, d_state):
        q, k, v, g, beta, ckpt = ctx.saved_tensors
        if d_o is None:
            d_o = torch.zeros(v.shape, device=v.device, dtype=torch.float32)
        need_ds0 = ctx.needs_input_grad[5]
        dq, dk, dv, dg, dbeta, ds0 = _chunkwise_backward(q, k, v, g, beta, ckpt, d_o, d_state, need_ds0)
        tq, tk, tv, tg, tb, ts = ctx.dtypes
        return (dq.to(tq), dk.to(tk), dv.to(tv), dg.to(tg), dbeta.to(tb),
                ds0.to(ts) if need_ds0 else None, None, None)


def kda_chunkwise(q, k, v, g, beta, initial_state=None, chunk_size=64, tile_size=0,
                  state_dtype=None):
    """Chunkwise KDA forward on gfx950 (signature of kimi_linear/kda.py:58-59).

    Returns ``(o [B, T, H, V] in v.dtype, state [B, H, K, V] in state_dtype or v.dtype)``.
    """
    del tile_size
    inputs = [x for x in (q, k, v, g, beta, initial_state) if isinstance(x, torch.Tensor)]
    if torch.is_grad_enabled() and any(x.requires_grad for x in inputs):
        K, V = q.shape[-1], v.shape[-1]
        if K not in (32, 64, 128) or V % BWD_TILE != 0:
            raise KdaError(f"the native chunkwise backward supports K in (32, 64, 128) and V a multiple "
                           f"of {BWD_TILE}; got K={K}, V={V} (call under torch.no_grad() for the forward)")
        return _ChunkwiseFn.apply(q, k, v, g, beta, initial_state, int(chunk_size), state_dtype)
    return _forward("chunkwise", q, k, v, g, beta, initial_state, int(chunk_size), state_dtype)


class _RecurrentFn(torch.autograd.Function):
    """kda_recurrent with a native backward.  The outputs come from the token
    kernel.  The gradient of the recurrence (``kda.py:196-219``) equals that of
    its chunkwise form (``kda.py:111-185``): the backward recomputes the
    chunkwise forward with checkpoints on the saved inputs and runs
    ``kda_chunkwise_bwd``.  An fp16 ``o`` was clamped to +-FP16_MAX_SAFE
    (``kda.py:217-218``): the gradient of a clamped (or NaN) entry is zero."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, state, state_dtype):
        o, s = _forward("recurrent", q, k, v, g, beta, state, 0, state_dtype)
        # differentiate what the backward kernels read: q, k in v's dtype, the gates in fp32
        ctx.save_for_backward(q.to(v.dtype), k.to(v.dtype), v, g.float(), beta.float(), state,
                              o if o.dtype is torch.float16 else None)
        ctx.state_dtype = state_dtype
        ctx.dtypes = (q.dtype, k.dtype, v.dtype, g.dtype, beta.dtype,
                      state.dtype if state is not None else None)
        return o, s

    @staticmethod
    def backward(ctx, d_o, d_state):
        q, k, v, g, beta, state, o16 = ctx.saved_tensors
        tq, tk, tv, tg, tb, ts = ctx.dtypes
        need_ds0 = ctx.needs_input_grad[5]
        B, T, H, K = q.shape
        V = v.shape[-1]
        if T == 0:
            zero = lambda shape, dt: torch.zeros(shape, device=q.device, dtype=dt)  # noqa: E731
            ds0 = None
            if need_ds0:
                ds0 = d_state.to(ts) if d_state is not None else zero((B, H, K, V), ts)
            return (zero(q.shape, tq), zero(k.shape, tk), zero(v.shape, tv), zero(g.shape, tg),
                    zero(beta.shape, tb), ds0, None)
        if d_o is None:
            d_o = torch.zeros(v.shape, device=v.device, dtype=torch.float32)
        elif o16 is not None:
            d_o = d_o * (o16.abs() < FP16_MAX_SAFE)
        _, _, ckpt = _forward("chunkwise", q, k, v, g, beta, state, 1, ctx.state_dtype, ckpt=True)
        dq, dk, dv, dg, dbeta, ds0 = _chunkwise_backward(q, k, v, g, beta, ckpt, d_o, d_state, need_ds0)
        return (dq.to(tq), dk.to(tk), dv.to(tv), dg.to(tg), dbeta.to(tb),
                ds0.to(ts) if need_ds0 else None, None)


def kda_recurrent(q, k, v, g, beta, state=None, state_dtype=None, *, state_out=None):
    """Token-by-token KDA recurrence on gfx950 (signature of kimi_linear/kda.py:188).

    Any ``T >= 0``; ``T == 1`` is the decode step.  Differentiable under grad
    mode (K in {32, 64, 128}, V a multiple of 32; see ``_RecurrentFn``).

    ``state_out`` (keyword-only, no counterpart in the reference) receives the
    new state instead of a fresh tensor: a contiguous ``[B, H, K, V]`` HIP
    tensor of dtype ``state_dtype or v.dtype``.  It may be ``state`` itself --
    an in-place update, which saves a decode loop with static state buffers
    (a captured graph) the copy of the whole state back into its input
    buffer.  It is returned as the second output.  Under autograd the state is
    always a new tensor: ``state_out`` is for loops that run without grad.
    """
    inputs = [x for x in (q, k, v, g, beta, state) if isinstance(x, torch.Tensor)]
    if torch.is_grad_enabled() and any(x.requires_grad for x in inputs):
        K, V = q.shape[-1], v.shape[-1]
        if state_out is not None:
            raise KdaError("state_out is an in-place update: kda_recurrent under autograd returns a new "
                           "state (call under torch.no_grad() or detach the inputs to use state_out)")
        if K not in (32, 64, 128) or V % BWD_TILE != 0:
            raise KdaError(f"the native backward supports K in (32, 64, 128) and V a multiple of "
                           f"{BWD_TILE}; got K={K}, V={V} (call under torch.no_grad() for the forward)")
        return _RecurrentFn.apply(q, k, v, g, beta, state, state_dtype)
    return _forward("recurrent", q, k, v, g, beta, state, 0, state_dtype, state_out)


def kda_chunkwise_gated(q, k, v, gk, beta_logit, a_log, dt_bias, initial_state=None, chunk_size=64,
                        state_dtype=None):
    """``kda_chunkwise`` with the KDA layer's gate pre-processing fused into the
    kernel's loads (no counterpart function in the reference; it computes
    ``g = -exp(A_log) * softplus(gk + dt_bias)`` and ``beta = sigmoid(beta_logit)``
    in fp32 as ``kimi_linear/kda.py:452-460`` does, then ``kda_chunkwise``).

    ``gk: [B, T, H, K]`` (the gate's up-projection), ``beta_logit: [B, T, H]``,
    ``a_log, dt_bias: [H, K]``.  For fp16 / bf16 q, k, v the gate inputs are read
    in that dtype (converted if they come in another); g and beta never exist
    in memory.  Forward only.  Returns ``(o, state)`` as ``kda_chunkwise``.
    """
    return _forward("chunkwise", q, k, v, gk, beta_logit, initial_state, int(chunk_size), state_dtype,
                    gate=(a_log, dt_bias))


def kda_recurrent_gated(q, k, v, gk, beta_logit, a_log, dt_bias, state=None, state_dtype=None, *,
                        state_out=None):
    """``kda_recurrent`` with the fused gate of :func:`kda_chunkwise_gated`
    (gate inputs in any float dtype).  ``state_out`` as in ``kda_recurrent``."""
    return _forward("recurrent", q, k, v, gk, beta_logit, state, 0, state_dtype, state_out, gate=(a_log, dt_bias))


def kda_chunkwise_fused(q, k, v, gk, beta_logit, a_log, dt_bias, og, norm_weight, eps, initial_state=None,
                        chunk_size=64, state_dtype=None):
    """:func:`kda_chunkwise_gated` with the KDA layer's output epilogue on the
    kernel's output tile (no counterpart function in the reference; it
    computes what ``_output`` does before ``o_proj``, ``kimi_linear/kda.py:
    258-279, 464-470``): ``y = x(x(rmsnorm(x(o)) * norm_weight) * sigmoid(og))``
    with x() the rounding to the activation dtype, as the reference's
    HeadwiseRMSNorm and output gate round.

    ``og: [B, T, H*V]`` (the output gate's up-projection), ``norm_weight:
    [H, V]``.  fp16 / bf16 q, k, v; K and V in (64, 128).  Forward only.
    Returns ``(y [B, T, H*V] in v.dtype, state)``.
    """
    o, s = _forward("chunkwise", q, k, v, gk, beta_logit, initial_state, int(chunk_size), state_dtype,
                    gate=(a_log, dt_bias), epilogue=(og, norm_weight, eps))
    B, T, H, V = o.shape
    return o.view(B, T, H * V), s
