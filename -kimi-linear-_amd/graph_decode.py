"""hipGraph-captured decoding over a stack of KDA layers.

The capture recipe of the reference's ``GraphedDecoder``
(``kimi_linear/graph_decode.py:241-289``), for the KDA part of the model:

* every layer's decode state (conv windows ``[B, conv_size - 1, D]`` and the
  fp32 recurrent state ``[B, H, K, V]``) lives in static buffers allocated
  after the eager prefill (``graph_decode.py:147-166``);
* warm-up runs of the step go on a side stream, then the graph is captured;
  both execute the step, so the post-prefill state is snapshotted before and
  restored after each (``graph_decode.py:268-289``);
* one replay is one complete decode step: the input is copied into a static
  buffer, the graph runs every layer, the output lands in a static buffer.

Where it differs: the reference's captured step ends with a copy of every
layer's new state back into the static buffers (``graph_decode.py:257-262``),
a full extra read and write of the 64 MiB-per-layer state (B=64, H=16,
K=V=128) each token.  Here the recurrence kernel updates the static state in
place (``KimiDeltaAttention.decode_step_``), so a replay touches each state
element exactly once for reading and once for writing; only the small conv
windows are shifted by copy.

The stack is ``h <- h + layer(h)`` per layer (``residual=True``) or
``h <- layer(h)``; the model's other blocks (MLA, FFN, norms, LM head) are not
part of the KDA path.
"""

from __future__ import annotations

from typing import Sequence

import torch
import torch.nn as nn

from .layer import KimiDeltaAttention


class KdaGraphedDecoder:
    """Graph-replayed incremental decoding of a stack of KDA layers.

    Usage::

        dec = KdaGraphedDecoder(layers)
        h = dec.prefill(x)           # [B, d], eager; (re)captures on a new batch size
        for _ in range(n):
            h = dec.step(x_t)        # x_t: [B, 1, d] -> [B, d], one graph replay

    ``step`` returns a view of the static output buffer: read or clone it
    before the next call.  Weights are read, never written, so one capture
    serves any number of prompts of the same batch size.

    The captured GEMMs read each layer's concatenated input-projection weight
    (``KimiDeltaAttention._input_weight``) and the parameters themselves, the
    gated recurrence the layer's fp32 copies of ``A_log`` and ``dt_bias``
    (``_gate_params``).  ``prefill`` refills these caches from the parameters
    (in place, so the graph keeps reading valid memory) and recaptures if a
    buffer had to be reallocated (new dtype or shape).  After updating weights between two
    ``step`` calls of one generation, call :meth:`refresh_weights`.
    """

    def __init__(self, layers: Sequence[KimiDeltaAttention], residual: bool = True, warmup_iters: int = 3):
        self.layers = nn.ModuleList(layers)
        if len(self.layers) == 0:
            raise ValueError("KdaGraphedDecoder needs at least one layer")
        self.layers.eval()
        self.residual = bool(residual)
        self.warmup_iters = int(warmup_iters)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.static_states: list[dict] | None = None
        self._B = None
        self._wbufs = None          # addresses of the fused weights the graph reads

    def _weight_buffers(self):
        bufs = []
        for layer in self.layers:
            w, b = layer._input_weight()
            a_log, dt_bias = layer._gate_params()
            bufs.append((w.data_ptr(), b.data_ptr() if b is not None else 0, a_log.data_ptr(), dt_bias.data_ptr()))
        return bufs

    @torch.no_grad()
    def refresh_weights(self) -> None:
        """Bring the captured step up to date with the layers' parameters:
        refill the fused input-projection weights and the fp32 gate
        parameters (in place) and recapture if one of them moved.  Needed only when weights change mid-generation."""
        if self.graph is None:
            return
        for layer in self.layers:
            layer.refresh_fused_weight()
        if self._weight_buffers() != self._wbufs:
            self._capture()

    # ------------------------------------------------------------ the stack
    def _run_stack(self, x, states, use_cache):
        h, new_states = x, []
        for layer, st in zip(self.layers, states):
            out, st_new = layer(h, state=st, use_cache=use_cache)
            new_states.append(st_new)
            h = h + out if self.residual else out
        return h, new_states

    @torch.no_grad()
    def _step(self):
        """The captured region: one token through every layer on the static buffers."""
        h = self.input_static
        for layer, st in zip(self.layers, self.static_states):
            out = layer.decode_step_(h, st)
            h = h + out if self.residual else out
        self.output_static.copy_(h[:, -1, :])

    # ------------------------------------------------------------ state plumbing
    def _snapshot(self):
        return [{"conv": {n: t.clone() for n, t in st["conv"].items()}, "recurrent": st["recurrent"].clone()}
                for st in self.static_states]

    def _restore(self, snap):
        for st, sn in zip(self.static_states, snap):
            for n in st["conv"]:
                st["conv"][n].copy_(sn["conv"][n])
            st["recurrent"].copy_(sn["recurrent"])

    def _fill_static(self, states):
        if self.static_states is None:
            self.static_states = [{"conv": {n: t.clone() for n, t in st["conv"].items()},
                                   "recurrent": st["recurrent"].clone()} for st in states]
        else:
            self._restore(states)

    @torch.no_grad()
    def _capture(self):
        torch.cuda.synchronize()
        snap = self._snapshot()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(self.warmup_iters):
                self._step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self._restore(snap)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()
        self._restore(snap)
        torch.cuda.synchronize()
        self._wbufs = self._weight_buffers()

    # ------------------------------------------------------------ public API
    @torch.no_grad()
    def prefill(self, x: torch.Tensor) -> torch.Tensor:
        """Eager prefill of ``x`` [B, S, d] (S >= 1) through the stack, then
        (re)capture.  Returns the last position's hidden state [B, d]."""
        if x.dim() != 3 or x.shape[1] < 1:
            raise ValueError(f"prefill takes x of shape [B, S >= 1, d], got {tuple(x.shape)}")
        if x.device.type != "cuda":
            raise ValueError("KdaGraphedDecoder runs on a HIP device")
        B = x.shape[0]
        h, states = self._run_stack(x, [None] * len(self.layers), use_cache=True)
        if self.graph is not None and B != self._B:
            self.graph = None
            self.static_states = None
        if self.static_states is not None and any(
                st["recurrent"].dtype != new["recurrent"].dtype for st, new in zip(self.static_states, states)):
            self.graph = None
            self.static_states = None
        if self.graph is not None and self._weight_buffers() != self._wbufs:
            self.graph = None           # a fused weight was reallocated: the graph would read freed memory
        self._fill_static(states)
        if self.graph is None:
            self._B = B
            self.input_static = torch.zeros(B, 1, x.shape[2], device=x.device, dtype=x.dtype)
            self.output_static = torch.empty(B, x.shape[2], device=x.device, dtype=x.dtype)
            self._capture()
        return h[:, -1, :]

    def step(self, x: torch.Tensor) -> torch.Tensor:
        """Advance one token: x [B, 1, d] -> [B, d] (a view of the static output)."""
        if self.graph is None:
            raise RuntimeError("call prefill() before step()")
        if tuple(x.shape) != tuple(self.input_static.shape):
            raise ValueError(f"step takes x of shape {tuple(self.input_static.shape)}, got {tuple(x.shape)}")
        self.input_static.copy_(x)
        self.graph.replay()
        return self.output_static

    @torch.no_grad()
    def step_eager(self, x: torch.Tensor) -> torch.Tensor:
        """The same step without the graph, on the same static state."""
        self.input_static.copy_(x)
        self._step()
        return self.output_static
