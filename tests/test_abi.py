"""CPU tests of the C ABI boundary: symbols, struct layout, host-side validation.

No kernel is launched here: every call below is rejected (or is empty) on the
host before the library touches the device.
"""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "kda_hip.h"


@pytest.fixture(scope="module")
def native(kda_pkg):
    import importlib
    mod = importlib.import_module("kimi_linear_amd._native")
    mod.load()
    return mod


def header_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(kda_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol(native):
    lib = native.load()
    declared = header_functions()
    assert declared == sorted(native.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name


def test_abi_version_and_status_strings(native):
    lib = native.load()
    assert lib.kda_abi_version() == native.ABI_VERSION
    for code in range(8):
        assert native.status_str(code)
    assert native.status_str(0) == "ok"
    assert "unknown" in native.status_str(99)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
@pytest.mark.parametrize("struct,cname", [("KdaFwdArgs", "kda_fwd_args"), ("KdaBwdArgs", "kda_bwd_args"),
                                          ("KdaGateArgs", "kda_gate_args"), ("KdaOutEpilogue", "kda_out_epilogue"),
                                          ("KdaPrepArgs", "kda_prep_args"),
                                          ("KdaOutputArgs", "kda_output_args"),
                                          ("KdaPrepBwdArgs", "kda_prep_bwd_args"),
                                          ("KdaOutputBwdArgs", "kda_output_bwd_args")])
def test_struct_layout_matches_header(native, tmp_path, struct, cname):
    cls = getattr(native, struct)
    fields = [name for name, _ in cls._fields_]
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "kda_hip.h"',
             "int main(void) {", f'  printf("size %zu\\n", sizeof({cname}));']
    lines += [f'  printf("{f} %zu\\n", offsetof({cname}, {f}));' for f in fields]
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", f"-I{HEADER.parent}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = dict(line.split() for line in out if line)
    assert int(got["size"]) == ctypes.sizeof(cls)
    for f in fields:
        assert int(got[f]) == getattr(cls, f).offset, f


def test_backward_workspace_size(native):
    """(K * V + 2 * 32 * V) floats per (b, h) and 32-token chunk (N is completed in
    the checkpoint records, not the workspace); 0 for bad shapes."""
    size = native.load().kda_chunkwise_bwd_workspace_size
    assert size(8, 4096, 16, 128, 128) == 8 * 16 * 128 * (128 * 128 + 64 * 128) * 4
    assert size(2, 80, 3, 64, 32) == 2 * 3 * 3 * (64 * 32 + 64 * 32) * 4    # ragged: 3 chunks
    assert size(1, 0, 1, 64, 64) == 0
    assert size(-1, 16, 1, 64, 64) == 0 and size(1, 16, 1, 0, 64) == 0


def test_backward_host_validation_codes(native):
    lib = native.load()

    def bargs(**kw):
        a = native.KdaBwdArgs()
        a.B, a.T, a.H, a.K, a.V = 1, 64, 1, 64, 64
        fake = 0x100000   # never dereferenced: every case here fails validation first
        for f in ("q", "k", "v", "g", "beta", "ckpt", "d_o", "dq", "dk", "dg", "dbeta", "dv", "workspace"):
            setattr(a, f, fake)
        a.scale, a.io_dtype = 0.125, native.DTYPE_F32
        for name, val in kw.items():
            setattr(a, name, val)
        return ctypes.byref(a)

    call = lib.kda_chunkwise_bwd
    assert call(None, None) == 1
    assert call(bargs(T=-1), None) == 2
    assert call(bargs(io_dtype=9), None) == 3
    assert call(bargs(K=48), None) == 4
    assert call(bargs(V=48), None) == 4
    assert call(bargs(workspace=None), None) == 1
    assert call(bargs(dq=None), None) == 1
    assert call(bargs(ckpt=None), None) == 1
    assert call(bargs(B=0), None) == 0                                   # empty: no launch
    assert call(bargs(T=0), None) == 0                                   # no d_state_in: nothing to do


def _args(native, **kw):
    a = native.KdaFwdArgs()
    a.B, a.T, a.H, a.K, a.V = 1, 16, 1, 64, 64
    fake = 0x100000   # never dereferenced: every case here fails validation first
    a.q = a.k = a.v = a.g = a.beta = a.o = fake
    a.state_out = fake * 4
    a.state_in = None
    a.chunk_size = 16
    a.scale = 0.125
    for name, val in kw.items():
        setattr(a, name, val)
    return a


@pytest.mark.parametrize("fn", ["kda_chunkwise_fwd", "kda_recurrent_fwd"])
def test_host_validation_codes(native, fn):
    lib = native.load()
    call = getattr(lib, fn)
    assert call(None, None) == 1                                          # NULL args
    assert call(ctypes.byref(_args(native, B=-1)), None) == 2            # bad shape
    assert call(ctypes.byref(_args(native, qkv_dtype=7)), None) == 3     # bad dtype
    assert call(ctypes.byref(_args(native, K=48)), None) == 4            # no kernel for K
    assert call(ctypes.byref(_args(native, q=None)), None) == 1          # missing input
    assert call(ctypes.byref(_args(native, state_out=None)), None) == 1
    overlap = _args(native)
    overlap.state_in = overlap.state_out + 8
    assert call(ctypes.byref(overlap), None) == 5                        # aliasing
    assert call(ctypes.byref(_args(native, B=0)), None) == 0             # empty: no launch
    assert call(ctypes.byref(_args(native, H=0)), None) == 0


@pytest.mark.parametrize("fn", ["kda_chunkwise_gated_fwd", "kda_recurrent_gated_fwd"])
def test_gated_host_validation_codes(native, fn):
    lib = native.load()
    call = getattr(lib, fn)
    gate = native.KdaGateArgs()
    gate.a_log, gate.dt_bias = 0x200000, 0x300000      # never dereferenced
    assert call(ctypes.byref(_args(native)), None, None) == 1              # no gate
    assert call(ctypes.byref(_args(native)), ctypes.byref(native.KdaGateArgs()), None) == 1
    assert call(ctypes.byref(_args(native, K=48)), ctypes.byref(gate), None) == 4
    assert call(ctypes.byref(_args(native, B=0)), ctypes.byref(native.KdaGateArgs()), None) == 0
    if fn == "kda_chunkwise_gated_fwd":
        # 16-bit q, k, v: the pipeline reads gk and the logits in that dtype
        bad = _args(native, qkv_dtype=native.DTYPE_F16, g_dtype=native.DTYPE_F32, beta_dtype=native.DTYPE_F16)
        assert call(ctypes.byref(bad), ctypes.byref(gate), None) == 3
        bad = _args(native, qkv_dtype=native.DTYPE_BF16, g_dtype=native.DTYPE_BF16, beta_dtype=native.DTYPE_F32)
        assert call(ctypes.byref(bad), ctypes.byref(gate), None) == 3


def test_fused_host_validation_codes(native):
    lib = native.load()
    call = lib.kda_chunkwise_fused_fwd
    gate = native.KdaGateArgs()
    gate.a_log, gate.dt_bias = 0x200000, 0x300000      # never dereferenced
    out = native.KdaOutEpilogue()
    out.gate, out.weight, out.eps = 0x400000, 0x500000, 1e-6
    out.gate_stride[0], out.gate_stride[1] = 16 * 64, 64
    f16 = dict(qkv_dtype=native.DTYPE_F16, g_dtype=native.DTYPE_F16, beta_dtype=native.DTYPE_F16)
    assert call(ctypes.byref(_args(native, **f16)), ctypes.byref(gate), None, None) == 1      # no epilogue
    assert call(ctypes.byref(_args(native)), ctypes.byref(gate), ctypes.byref(out), None) == 4  # fp32: no kernel
    assert call(ctypes.byref(_args(native, V=96, **f16)), ctypes.byref(gate), ctypes.byref(out), None) == 4
    assert call(ctypes.byref(_args(native, T=20, **f16)), ctypes.byref(gate), ctypes.byref(out), None) == 2
    bad = native.KdaOutEpilogue()
    bad.gate, bad.weight, bad.eps = 0x400000, 0x500000, -1.0
    assert call(ctypes.byref(_args(native, **f16)), ctypes.byref(gate), ctypes.byref(bad), None) == 2
    nog = native.KdaOutEpilogue()
    nog.eps = 1e-6
    assert call(ctypes.byref(_args(native, **f16)), ctypes.byref(gate), ctypes.byref(nog), None) == 1
    assert call(ctypes.byref(_args(native, B=0, **f16)), ctypes.byref(gate), ctypes.byref(out), None) == 0


def test_long_host_validation_codes(native):
    lib = native.load()
    call = lib.kda_chunkwise_long_fwd
    f16 = dict(qkv_dtype=native.DTYPE_F16, T=64, chunk_size=16)
    assert call(ctypes.byref(_args(native, **f16)), 0, None, None) == 2            # no segments
    assert call(ctypes.byref(_args(native, **f16)), 3, None, None) == 2            # T % segments
    assert call(ctypes.byref(_args(native, T=64, chunk_size=16)), 2, None, None) == 4  # fp32: no split kernel
    assert call(ctypes.byref(_args(native, K=32, **f16)), 2, None, None) == 4
    assert call(ctypes.byref(_args(native, **f16)), 2, None, None) == 1            # no workspace
    assert call(ctypes.byref(_args(native, **f16)), 2, ctypes.c_void_p(0x100008), None) == 2  # misaligned
    assert call(ctypes.byref(_args(native, B=0, **f16)), 2, None, None) == 0
    size = lib.kda_chunkwise_long_workspace_size
    # per segment and head: S_loc and Phi (K x (V + K)) and the initial state (K x V), fp32
    # 16 segments of 16 heads: the first pass takes two rounds of 128-column
    # workgroups (three passes); 8 segments: one round (the few-chain form,
    # which also keeps the fp32 outputs and their initial-state coefficients)
    assert size(1, 32768, 16, 128, 128, 16) == 4 * 16 * 16 * 128 * (2 * 128 + 128)
    assert size(1, 32768, 16, 128, 128, 8) == 4 * (8 * 16 * 128 * (2 * 128 + 128) + 32768 * 16 * (128 + 128))
    assert size(1, 64, 1, 64, 64, 0) == 0


def test_in_place_state_contract(native):
    lib = native.load()
    same = _args(native, K=48)           # K=48 has no kernel: validation ends before any launch
    same.state_in = same.state_out
    # the recurrence accepts an exact alias (in-place update) and gets as far as the head-size check
    assert lib.kda_recurrent_fwd(ctypes.byref(same), None) == 4
    # the chunkwise pipeline does not, nor does an alias that changes dtype
    assert lib.kda_chunkwise_fwd(ctypes.byref(same), None) == 5
    same.state_in_dtype = native.DTYPE_F16
    assert lib.kda_recurrent_fwd(ctypes.byref(same), None) == 5


def test_chunkwise_row_stride_contract(native):
    # chunkwise reads each chunk through a descriptor spanning its token rows,
    # so a token stride shorter than a row is rejected before any launch
    lib = native.load()
    good = dict(q_stride=(ctypes.c_int64 * 3)(16 * 64, 64, 64), k_stride=(ctypes.c_int64 * 3)(16 * 64, 64, 64),
                v_stride=(ctypes.c_int64 * 3)(16 * 64, 64, 64), g_stride=(ctypes.c_int64 * 3)(16 * 64, 64, 64),
                beta_stride=(ctypes.c_int64 * 3)(16, 1, 1))
    for name, bad in (("q_stride", (16 * 64, 0, 64)), ("g_stride", (16 * 64, 32, 64)),
                      ("v_stride", (16 * 64, 63, 64)), ("beta_stride", (16, 0, 1))):
        kw = dict(good)
        kw[name] = (ctypes.c_int64 * 3)(*bad)
        assert lib.kda_chunkwise_fwd(ctypes.byref(_args(native, **kw)), None) == 4, name


def test_chunk_contract(native):
    lib = native.load()
    assert lib.kda_chunkwise_fwd(ctypes.byref(_args(native, T=20, chunk_size=16)), None) == 2
    assert lib.kda_chunkwise_fwd(ctypes.byref(_args(native, chunk_size=0)), None) == 2
    # the recurrence ignores chunk_size
    assert lib.kda_recurrent_fwd(ctypes.byref(_args(native, T=20, chunk_size=16, K=48)), None) == 4


def test_wrapper_rejects_cpu_tensors(kda_pkg):
    B, T, H, K, V = 1, 16, 1, 64, 64
    q = torch.zeros(B, T, H, K)
    beta = torch.zeros(B, T, H)
    with pytest.raises(kda_pkg.KdaError, match="no CPU path"):
        kda_pkg.kda_chunkwise(q, q, torch.zeros(B, T, H, V), q, beta, chunk_size=16)
    with pytest.raises(kda_pkg.KdaError, match="no CPU path"):
        kda_pkg.kda_recurrent(q, q, torch.zeros(B, T, H, V), q, beta)


def test_wrapper_shape_and_chunk_errors(kda_pkg):
    q = torch.zeros(1, 20, 1, 64)
    beta = torch.zeros(1, 20, 1)
    v = torch.zeros(1, 20, 1, 64)
    with pytest.raises(ValueError, match="multiple of chunk_size"):
        kda_pkg.kda_chunkwise(q, q, v, q, beta, chunk_size=16)
    with pytest.raises(RuntimeError):       # the reference's reshape raises RuntimeError
        kda_pkg.kda_chunkwise(q, q, v, q, beta, chunk_size=16)
    with pytest.raises(kda_pkg.KdaError, match="beta must be"):
        kda_pkg.kda_recurrent(q, q, v, q, torch.zeros(1, 20, 2))
    with pytest.raises(kda_pkg.KdaError, match="state must be"):
        kda_pkg.kda_recurrent(q, q, v, q, beta, state=torch.zeros(1, 1, 64, 32))


def test_layer_training_path_refuses_head_dims_its_backward_lacks(kda_pkg):
    """value_head_dim 256 has a forward but no pre-processing backward: the
    training path refuses it before any work (here on CPU tensors, which
    would fail later anyway)."""
    cfg = kda_pkg.linear_attn_config(hidden_size=256, num_heads=1, head_dim=128, value_head_dim=256,
                                     gate_low_rank=32, output_gate_low_rank=32)
    m = kda_pkg.KimiDeltaAttention(cfg)
    x = torch.zeros(1, 8, 256, requires_grad=True)
    with pytest.raises(kda_pkg.KdaError, match="training path supports head_dim"):
        m(x)


def test_noalloc_backward_rejects_shapes_beyond_its_buffer(native):
    """kda_chunkwise_bwd_noalloc refuses, on the host and before touching the
    device, a shape whose workspace exceeds KDA_BWD_SCRATCH_BYTES."""
    lib = native.load()
    header = HEADER.read_text()
    assert re.search(r"#define KDA_BWD_SCRATCH_BYTES \(\(size_t\)64 << 20\)", header)
    assert native.BWD_SCRATCH_BYTES == 64 << 20
    a = native.KdaBwdArgs()
    a.B, a.T, a.H, a.K, a.V = 8, 4096, 16, 128, 128
    assert lib.kda_chunkwise_bwd_workspace_size(8, 4096, 16, 128, 128) > native.BWD_SCRATCH_BYTES
    fake = 0x1000                       # never dereferenced: the call is rejected first
    for f in ("q", "k", "v", "g", "beta", "ckpt", "d_o", "dq", "dk", "dg", "dbeta", "dv"):
        setattr(a, f, fake)
    a.io_dtype = native.DTYPE_F16
    a.workspace = None                  # ignored by the no-allocation entry point
    assert lib.kda_chunkwise_bwd_noalloc(ctypes.byref(a), None) == native.STATUS_TOO_LARGE
    a.q = None
    assert lib.kda_chunkwise_bwd_noalloc(ctypes.byref(a), None) == 1     # NULL input first
    a.B = 0
    assert lib.kda_chunkwise_bwd_noalloc(ctypes.byref(a), None) == 0     # empty: nothing to do


def test_layer_backward_workspace_sizes(native):
    """prep: per 64-token tile, every conv channel's taps and bias plus two gate
    parameters per q/k channel (fp32); output: per 32-token tile, H * V."""
    lib = native.load()
    assert lib.kda_prep_bwd_workspace_size(2, 130, 4, 64, 128, 4) == 2 * 3 * ((2 * 256 + 512) * 5 + 2 * 256) * 4
    assert lib.kda_prep_bwd_workspace_size(1, 0, 4, 64, 64, 4) == 0
    assert lib.kda_prep_bwd_workspace_size(1, 16, 4, 64, 64, 0) == 0
    assert lib.kda_output_bwd_workspace_size(2, 33, 4, 64) == 2 * 2 * 4 * 64 * 4
    assert lib.kda_output_bwd_workspace_size(2, 0, 4, 64) == 0


def test_layer_backward_host_validation_codes(native):
    lib = native.load()
    fake = 0x100000   # never dereferenced: every case here fails validation first

    def pargs(**kw):
        a = native.KdaPrepBwdArgs()
        a.B, a.T, a.H, a.K, a.V, a.conv_size = 1, 64, 2, 64, 64, 4
        for i in range(3):
            a.x[i] = a.conv_w[i] = a.dy[i] = a.dx[i] = a.dw[i] = fake
        a.workspace = fake
        a.l2_eps, a.x_dtype, a.w_dtype = 1e-6, native.DTYPE_F16, native.DTYPE_F32
        for name, val in kw.items():
            setattr(a, name, val)
        return ctypes.byref(a)

    call = lib.kda_prep_bwd
    assert call(None, None) == 1
    assert call(pargs(T=-1), None) == 2
    assert call(pargs(K=32), None) == 4 and call(pargs(V=256), None) == 4
    assert call(pargs(conv_size=5), None) == 4
    assert call(pargs(x_dtype=9), None) == 3
    assert call(pargs(l2_eps=0.0), None) == 2
    assert call(pargs(workspace=None), None) == 1
    assert call(pargs(gk=fake), None) == 1            # gates without their other pointers
    assert call(pargs(T=0), None) == 0                # nothing to do

    def oargs(**kw):
        a = native.KdaOutputBwdArgs()
        a.B, a.T, a.H, a.V = 1, 8, 2, 64
        for f in ("o", "gate", "weight", "dy", "d_o", "dgate", "dweight", "workspace"):
            setattr(a, f, fake)
        a.eps, a.x_dtype, a.w_dtype = 1e-6, native.DTYPE_F16, native.DTYPE_F32
        for name, val in kw.items():
            setattr(a, name, val)
        return ctypes.byref(a)

    call = lib.kda_output_bwd
    assert call(None, None) == 1
    assert call(oargs(V=96), None) == 4
    assert call(oargs(w_dtype=7), None) == 3
    assert call(oargs(eps=-1.0), None) == 2
    assert call(oargs(dweight=None), None) == 1
    assert call(oargs(T=0), None) == 0
