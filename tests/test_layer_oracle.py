"""Pins of the KDA-layer oracle (CPU): textbook references for its pieces and
invariances of the whole layer's dispatch and cache handling."""

from __future__ import annotations

import math
from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F

from oracle.kda_layer_oracle import (head_rmsnorm_ref, kda_layer_ref, l2norm_ref, make_layer_params,
                                     short_conv_ref)


def small_cfg(**kw):
    la = dict(num_heads=2, head_dim=32, value_head_dim=32, conv_size=4, chunk_size=16, tile_size=0,
              proj_bias=False, conv_bias=True, gate_low_rank=16, output_gate_low_rank=16,
              a_log_init=0.0, dt_bias_init=0.0)
    la.update(kw)
    return SimpleNamespace(linear_attn_config=la, hidden_size=64, l2norm_eps=1e-6, rms_norm_eps=1e-6)


def test_short_conv_matches_conv1d():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 11, 6, generator=g)
    w = torch.randn(6, 1, 4, generator=g)
    b = torch.randn(6, generator=g)
    ref = F.conv1d(F.pad(x.transpose(1, 2), (3, 0)), w, b, groups=6).transpose(1, 2)
    assert torch.allclose(short_conv_ref(x, w, b), ref, atol=1e-6)
    # history of earlier inputs == convolving the concatenation and dropping the prefix
    h = torch.randn(2, 3, 6, generator=g)
    full = F.conv1d(F.pad(torch.cat([h, x], 1).transpose(1, 2), (3, 0)), w, b, groups=6).transpose(1, 2)
    assert torch.allclose(short_conv_ref(x, w, b, history=h), full[:, 3:], atol=1e-6)


def test_norms_match_torch():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 5, 2, 8, generator=g)
    x[0, 0, 0] = 0.0                                   # the eps clamp keeps zero rows finite
    assert torch.allclose(l2norm_ref(x, 1e-6), F.normalize(x, dim=-1, eps=1e-6), atol=1e-6)
    w = torch.randn(2, 8, generator=g)
    assert torch.allclose(head_rmsnorm_ref(x, w, 1e-6), F.rms_norm(x, (8,), eps=1e-6) * w, atol=1e-6)


def test_chunked_prefill_and_decode_equal_one_pass():
    cfg = small_cfg()
    p = make_layer_params(cfg, seed=2)
    x = torch.randn(2, 45, 64, generator=torch.Generator().manual_seed(3))
    full = kda_layer_ref(p, cfg, x)
    # chunked prefill through the conv cache and recurrent state
    o1, st = kda_layer_ref(p, cfg, x[:, :20], use_cache=True)
    o2, st = kda_layer_ref(p, cfg, x[:, 20:37], state=st, use_cache=True)
    outs = [o1, o2]
    # then token by token (the T == 1 cached path)
    for t in range(37, 45):
        o, st = kda_layer_ref(p, cfg, x[:, t:t + 1], state=st, use_cache=True)
        outs.append(o)
    assert torch.allclose(torch.cat(outs, 1), full, atol=2e-5, rtol=1e-4)


def test_chunk_size_and_tail_split_do_not_matter():
    x = torch.randn(1, 37, 64, generator=torch.Generator().manual_seed(4))
    p = make_layer_params(small_cfg(), seed=5)
    base = kda_layer_ref(p, small_cfg(chunk_size=16), x)          # body 32 + tail 5
    for c in (8, 37, 64):                                          # 64 > T: one chunk of T
        assert torch.allclose(kda_layer_ref(p, small_cfg(chunk_size=c), x), base, atol=2e-5, rtol=1e-4)


def test_decode_from_empty_state_equals_prefill():
    cfg = small_cfg()
    p = make_layer_params(cfg, seed=6)
    x = torch.randn(3, 6, 64, generator=torch.Generator().manual_seed(7))
    full = kda_layer_ref(p, cfg, x)
    st, outs = None, []
    for t in range(6):
        o, st = kda_layer_ref(p, cfg, x[:, t:t + 1], state=st, use_cache=True)
        outs.append(o)
    assert torch.allclose(torch.cat(outs, 1), full, atol=2e-5, rtol=1e-4)
    assert st["conv"]["q"].shape == (3, 3, 64) and st["recurrent"].shape == (3, 2, 32, 32)


# ------------------------------------------------------------- host-side module pieces
def test_module_parameters_match_reference_names(kda_pkg):
    cfg = small_cfg()
    m = kda_pkg.KimiDeltaAttention(cfg)
    p = make_layer_params(cfg, seed=8)
    sd = m.state_dict()
    assert set(sd) == set(p)
    assert all(sd[n].shape == p[n].shape for n in p)
    m.load_state_dict(p)


def test_module_core_needs_hip_device(kda_pkg):
    """The layer's core runs only on the HIP kernels: CPU tensors raise."""
    m = kda_pkg.KimiDeltaAttention(small_cfg())
    with torch.no_grad(), pytest.raises(kda_pkg.KdaError):
        m(torch.randn(1, 16, 64))
