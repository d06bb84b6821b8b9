"""CPU tests of the layer's callable helper modules -- ``ShortConv``,
``HeadwiseRMSNorm`` and ``l2norm`` (``kimi_linear/kda.py:258-325``) -- for
reference-side code that calls them directly.  The checkers are the layer
oracle's pieces, which tests/test_layer_oracle.py pins against
``F.conv1d`` with history, ``F.rms_norm`` and ``F.normalize``."""

from __future__ import annotations

import pytest
import torch

from oracle.kda_layer_oracle import head_rmsnorm_ref, l2norm_ref, short_conv_ref


def _rel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm()).item()


@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("cs", [4, 2])
def test_short_conv_forward_and_cached_step(kda_pkg, bias, cs):
    torch.manual_seed(cs + bias)
    B, T, D = 2, 21, 48
    m = kda_pkg.ShortConv(D, cs, bias=bias)
    x = torch.randn(B, T, D)
    with torch.no_grad():
        y = m(x)
        ref = short_conv_ref(x, m.conv.weight, m.conv.bias)
        assert y.shape == (B, T, D) and _rel(y, ref) <= 1e-6
        # one cached token continues the sequence: the window is the last cs - 1 inputs + x_t
        state = x[:, T - cs:T - 1] if cs > 1 else x[:, :0]
        yt, new_state = m(x[:, T - 1:T], state, use_cache=True)
        assert yt.shape == (B, 1, D) and _rel(yt[:, 0], ref[:, T - 1]) <= 1e-6
        assert torch.equal(new_state, x[:, T - cs + 1:T])
        # fp16 inputs keep their dtype, the cached sum runs in fp32
        yh, _ = m.half()(x[:, :1].half(), state[:, :cs - 1].half(), use_cache=True)
        assert yh.dtype == torch.float16


def test_headwise_rmsnorm_forward(kda_pkg):
    torch.manual_seed(3)
    B, T, H, D = 2, 5, 3, 32
    m = kda_pkg.HeadwiseRMSNorm(H, D, 1e-6)
    with torch.no_grad():
        m.weight.normal_(1.0, 0.1)
    x = torch.randn(B, T, H, D)
    with torch.no_grad():
        assert _rel(m(x), head_rmsnorm_ref(x, m.weight, 1e-6)) <= 1e-6
        assert m(x.half()).dtype == torch.float16


def test_l2norm(kda_pkg):
    torch.manual_seed(4)
    x = torch.randn(3, 7, 2, 64)
    assert _rel(kda_pkg.l2norm(x, 1e-6), l2norm_ref(x, 1e-6)) <= 1e-6
    tiny = torch.full((1, 64), 1e-9)                      # rsqrt clamped to 1 / eps
    assert torch.allclose(kda_pkg.l2norm(tiny, 1e-6), tiny * 1e6)
    assert kda_pkg.l2norm(x.half(), 1e-6).dtype == torch.float16
