"""The layer oracle against the reference module's own outputs (CPU).

``tests/golden/kda_layer_golden.pt`` holds weights, inputs, outputs and states
that ``tests/golden/make_layer_golden.py`` wrote by running the reference's
``KimiDeltaAttention`` (kimi_linear/kda.py:331-536) in fp32 on the CPU: one-pass
prefill with a recurrent tail, the same with a cache, a sequence shorter than a
chunk, chunked prefill from a cached state, and single-token decode steps.  The
oracle ``kda_layer_ref`` must reproduce every output and every state.

Mutations of the oracle that a transcription slip could make (conv taps in the
wrong order, SiLU or the L2 norm left out, the head norm's weight dropped,
softplus replaced) must each break the match: the fixture pins
the composition, not only the pieces.
"""

from __future__ import annotations

import pytest
import torch

from oracle import kda_layer_oracle as klo
from tests.golden import CASES, load_fixture, shape_config, shape_params, state_of

TOL = 2e-5       # relative L2, fp32 vs fp32 (different summation orders only)


@pytest.fixture(scope="module")
def golden():
    return load_fixture()


def rel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm()).item()


def run_case(data, name, case):
    """The oracle on one fixture case; returns {key: tensor} like the fixture's."""
    cfg = shape_config(data["meta"], name)
    p = shape_params(data, name)
    pre = f"{name}."
    if case == "prefill":
        return {"out": klo.kda_layer_ref(p, cfg, data[pre + "prefill.x"])}
    if case == "prefill_c":
        out, st = klo.kda_layer_ref(p, cfg, data[pre + "prefill.x"], use_cache=True)
    elif case == "short":
        out, st = klo.kda_layer_ref(p, cfg, data[pre + "short.x"], use_cache=True)
    elif case == "chunked":
        st0 = state_of(data, pre + "prefill_c.state")
        out, st = klo.kda_layer_ref(p, cfg, data[pre + "chunked.x"], state=st0, use_cache=True)
    else:
        st = state_of(data, pre + "chunked.state")
        x = data[pre + "decode.x"]
        outs = []
        for t in range(x.shape[1]):
            o, st = klo.kda_layer_ref(p, cfg, x[:, t:t + 1], state=st, use_cache=True)
            outs.append(o)
        out = torch.cat(outs, 1)
    res = {"out": out, "state.recurrent": st["recurrent"]}
    res.update({f"state.conv.{n}": st["conv"][n] for n in ("q", "k", "v")})
    return res


def case_errors(data, name, case):
    got = run_case(data, name, case)
    return {k: rel(v, data[f"{name}.{case}.{k}"].float()) for k, v in got.items()}


def test_fixture_manifest(golden):
    meta = golden["meta"]
    assert set(meta["shapes"]) == {"tiny", "k64"}
    tiny = meta["shapes"]["tiny"]["linear_attn"]
    # the reference's tiny test configuration, unchanged
    assert (tiny["num_heads"], tiny["head_dim"], tiny["chunk_size"], tiny["conv_size"]) == (2, 32, 16, 4)
    for name in meta["shapes"]:
        for case in CASES:
            assert torch.isfinite(golden[f"{name}.{case}.out"]).all()


@pytest.mark.parametrize("name", ["tiny", "k64"])
@pytest.mark.parametrize("case", CASES)
def test_layer_oracle_matches_reference_outputs(golden, name, case):
    errs = case_errors(golden, name, case)
    assert max(errs.values()) <= TOL, errs


def _flip_taps(fn):
    def conv(x, weight, bias=None, history=None):
        return fn(x, weight.flip(-1), bias, history)
    return conv


MUTATIONS = {
    "conv taps reversed": ("short_conv_ref", lambda f: _flip_taps(f)),
    "no SiLU": ("_silu", lambda f: (lambda x: x)),
    "no L2 norm": ("l2norm_ref", lambda f: (lambda x, eps: x.float())),
    "head norm without weight": ("head_rmsnorm_ref", lambda f: (lambda x, w, eps: f(x, torch.ones_like(w), eps))),
    "softplus -> relu": ("_softplus", lambda f: (lambda x: torch.relu(x))),
}


@pytest.mark.parametrize("mutation", list(MUTATIONS))
def test_fixture_catches_oracle_mutations(golden, monkeypatch, mutation):
    """A plausible slip in the oracle fails at least one fixture case by far
    more than the tolerance."""
    attr, make = MUTATIONS[mutation]
    monkeypatch.setattr(klo, attr, make(getattr(klo, attr)))
    worst = max(max(case_errors(golden, "k64", case).values()) for case in ("prefill", "decode"))
    assert worst > 100 * TOL, f"{mutation}: fixture error only {worst:.2e}"
