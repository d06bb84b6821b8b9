"""The HIP KDA layer against the reference module's own outputs.

The "k64" shape of ``tests/golden/kda_layer_golden.pt`` (hidden 64, 2 heads x 64,
chunk 16, conv 4, projection and conv biases) was written by the reference's
``KimiDeltaAttention`` in fp32 (see ``tests/golden/make_layer_golden.py``).
Its weights load into ``kimi_linear_amd.KimiDeltaAttention`` through
``load_state_dict`` with the reference's key names (strict), and every case --
prefill with a recurrent tail, with and without a cache, T < chunk, chunked
prefill from a cached state, three decode steps -- must reproduce the
reference's outputs and states.  Tolerance (relative L2): fp32 2e-5 (fp32
throughout), fp16 5e-3 (fp16 activations round every projection to 11 bits).
"""

from __future__ import annotations

import pytest
import torch

from tests.golden import load_fixture, shape_config, shape_params, state_of

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL = {torch.float32: 2e-5, torch.float16: 5e-3}


@pytest.fixture(scope="module")
def golden():
    return load_fixture()


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm()).item()


def to_dev(st, dtype):
    return {"conv": {n: t.to(DEV, dtype) for n, t in st["conv"].items()},
            "recurrent": st["recurrent"].to(DEV, torch.float32)}


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_hip_layer_matches_reference_outputs(kda_pkg, golden, dtype):
    cfg = shape_config(golden["meta"], "k64")
    m = kda_pkg.KimiDeltaAttention(cfg)
    m.load_state_dict(shape_params(golden, "k64"), strict=True)
    m = m.to(DEV, dtype).eval()
    tol = TOL[dtype]

    def x_of(case):
        return golden[f"k64.{case}.x"].to(DEV, dtype)

    def check(case, out, st=None):
        errs = {"out": rel(out, golden[f"k64.{case}.out"])}
        if st is not None:
            ref = state_of(golden, f"k64.{case}.state")
            errs["recurrent"] = rel(st["recurrent"], ref["recurrent"])
            for n in ("q", "k", "v"):
                errs[f"conv.{n}"] = rel(st["conv"][n], ref["conv"][n])
        print(f"golden k64 {dtype} {case}: " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
        assert max(errs.values()) <= tol, (case, errs)

    with torch.no_grad():
        check("prefill", m(x_of("prefill")))
        out, st = m(x_of("prefill"), use_cache=True)
        check("prefill_c", out, st)
        out, st = m(x_of("short"), use_cache=True)
        check("short", out, st)
        out, st = m(x_of("chunked"), state=to_dev(state_of(golden, "k64.prefill_c.state"), dtype), use_cache=True)
        check("chunked", out, st)
        st = to_dev(state_of(golden, "k64.chunked.state"), dtype)
        xd = x_of("decode")
        outs = []
        for t in range(xd.shape[1]):
            o, st = m(xd[:, t:t + 1], state=st, use_cache=True)
            outs.append(o)
        check("decode", torch.cat(outs, 1), st)
