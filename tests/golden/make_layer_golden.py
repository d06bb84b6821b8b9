"""Write the KDA-layer golden fixture from the reference module itself.

Runs ONLY in the build container, where the reference checkout sits at
/root/reference: it imports ``kimi_linear`` there (CPU, fp32), runs
``KimiDeltaAttention.forward`` (kimi_linear/kda.py:473-536) in every mode its
dispatch has, and saves plain tensors -- weights, inputs, outputs, states -- to
``kda_layer_golden.pt`` beside this script.  Nothing of the reference travels
with the fixture: it holds numbers only, and tests load it with
``torch.load(..., weights_only=True)``.

Why a fixture: the layer composition (projection order, where SiLU, the L2
norm, the gates and the head-wise norm sit, the softplus argument, the cached
conv window, the chunk/tail dispatch) is restated by the layer oracle, and no
closed form pins that composition.  The core kernels (``kda_chunkwise``,
``kda_recurrent``) are pinned by closed forms and by the fp64 matrix form of
the recurrence, so no core vectors are written here; the layer cases run
through them anyway.

Two layer shapes:
  * "tiny": the reference's own ``configs/kimi_linear_tiny_test.json``
    linear-attention block (hidden 64, 2 heads x 32, chunk 16, conv 4, conv
    bias, no projection bias);
  * "k64": hidden 64, 2 heads x 64, chunk 16, conv 4, with projection and conv
    biases -- head dims the HIP layer kernels take, so the GPU test can run it.

Cases per shape (x ~ N(0, 1), weights as in ``make_params``):
  prefill      T=40 without cache (body 32 chunkwise + tail 8 recurrent)
  prefill_c    the same x with use_cache from an empty state -> out, state
  short        T=10 < chunk with use_cache -> out, state
  chunked      T=21 continuing from prefill_c's state -> out, state
  decode       3 single-token steps continuing from chunked's state

Usage: python tests/golden/make_layer_golden.py
"""

from __future__ import annotations

import json
import math
import sys
from pathlib import Path
from types import SimpleNamespace

import torch

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "kda_layer_golden.pt"


def tiny_linear_attn() -> dict:
    with open(REF / "configs" / "kimi_linear_tiny_test.json", encoding="utf-8") as f:
        doc = json.load(f)
    return dict(doc["linear_attn"]), doc


def make_params(la: dict, d: int, seed: int) -> dict:
    """Weights with the reference's parameter names: projections N(0, 0.1)
    (large enough that every path moves the output), conv taps N(0, 0.3),
    biases N(0, 0.05), A_log ~ U(0, ln 16), dt_bias ~ N(0, 0.1), norm weight
    1 + N(0, 0.1)."""
    H, K, V, C = la["num_heads"], la["head_dim"], la["value_head_dim"], la["conv_size"]
    gen = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    p = {}

    def lin(name, i, o):
        p[name + ".weight"] = rn(o, i) * (1.0 / math.sqrt(i))
        if la["proj_bias"]:
            p[name + ".bias"] = rn(o) * 0.05

    lin("in_proj_q", d, H * K)
    lin("in_proj_k", d, H * K)
    lin("in_proj_v", d, H * V)
    for n, dim in (("q", H * K), ("k", H * K), ("v", H * V)):
        p[f"conv_{n}.conv.weight"] = rn(dim, 1, C) * 0.3
        if la["conv_bias"]:
            p[f"conv_{n}.conv.bias"] = rn(dim) * 0.05
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


def clone_state(st):
    return {"conv": {n: t.clone() for n, t in st["conv"].items()},
            "recurrent": None if st["recurrent"] is None else st["recurrent"].clone()}


def flat_state(prefix: str, st: dict, out: dict) -> None:
    for n, t in st["conv"].items():
        out[f"{prefix}.conv.{n}"] = t.detach().clone().contiguous()
    out[f"{prefix}.recurrent"] = st["recurrent"].detach().clone().contiguous()


def run_shape(KDA, name: str, la: dict, d: int, eps: dict, seed: int) -> dict:
    cfg = SimpleNamespace(linear_attn_config=la, hidden_size=d, **eps)
    layer = KDA(cfg).eval()
    params = make_params(la, d, seed)
    layer.load_state_dict(params, strict=True)
    gen = torch.Generator().manual_seed(seed + 100)
    B = 2
    x40 = torch.randn(B, 40, d, generator=gen)
    x10 = torch.randn(B, 10, d, generator=gen)
    x21 = torch.randn(B, 21, d, generator=gen)
    xdec = torch.randn(B, 3, d, generator=gen)
    rec = {}
    with torch.no_grad():
        rec["prefill.x"] = x40
        rec["prefill.out"] = layer(x40)
        out, st = layer(x40, use_cache=True)
        rec["prefill_c.out"] = out
        flat_state("prefill_c.state", st, rec)
        rec["short.x"] = x10
        out_s, st_s = layer(x10, use_cache=True)
        rec["short.out"] = out_s
        flat_state("short.state", st_s, rec)
        rec["chunked.x"] = x21
        out_c, st_c = layer(x21, state=clone_state(st), use_cache=True)
        rec["chunked.out"] = out_c
        flat_state("chunked.state", st_c, rec)
        rec["decode.x"] = xdec
        st_d = clone_state(st_c)
        outs = []
        for t in range(xdec.shape[1]):
            o, st_d = layer(xdec[:, t:t + 1], state=st_d, use_cache=True)
            outs.append(o)
        rec["decode.out"] = torch.cat(outs, 1)
        flat_state("decode.state", st_d, rec)
    fixture = {f"{name}.param.{k}": v.detach().clone().contiguous() for k, v in params.items()}
    fixture.update({f"{name}.{k}": v.detach().clone().contiguous() for k, v in rec.items()})
    return fixture


def main() -> None:
    if not (REF / "kimi_linear" / "kda.py").exists():
        raise SystemExit(f"the reference checkout is not at {REF}: this script only runs in the build container")
    sys.path.insert(0, str(REF))
    from kimi_linear.kda import KimiDeltaAttention  # noqa: E402  (the reference module)

    torch.set_default_dtype(torch.float32)
    la_tiny, doc = tiny_linear_attn()
    eps = {"l2norm_eps": float(doc["l2norm_eps"]), "rms_norm_eps": float(doc["rms_norm_eps"])}
    la_k64 = dict(la_tiny, head_dim=64, value_head_dim=64, proj_bias=True, conv_bias=True)
    shapes = {"tiny": (la_tiny, int(doc["hidden_size"]), 0), "k64": (la_k64, int(doc["hidden_size"]), 1)}
    fixture = {}
    meta = {"torch": torch.__version__, "generated_by": "tests/golden/make_layer_golden.py",
            "dtype": "float32", "device": "cpu", "shapes": {}}
    for name, (la, d, seed) in shapes.items():
        fixture.update(run_shape(KimiDeltaAttention, name, la, d, eps, seed))
        meta["shapes"][name] = {"linear_attn": la, "hidden_size": d, "seed": seed, **eps}
    fixture["meta_json"] = json.dumps(meta, sort_keys=True)
    torch.save(fixture, OUT)
    n = sum(v.numel() for v in fixture.values() if isinstance(v, torch.Tensor))
    print(f"wrote {OUT} ({n} values, {OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
