"""Golden fixtures written from the reference module (see make_layer_golden.py)."""

from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace

import torch

FIXTURE = Path(__file__).resolve().parent / "kda_layer_golden.pt"
CASES = ("prefill", "prefill_c", "short", "chunked", "decode")


def load_fixture() -> dict:
    """The fixture as a dict of tensors plus ``meta`` (parsed JSON); no code is loaded."""
    data = torch.load(FIXTURE, map_location="cpu", weights_only=True)
    data["meta"] = json.loads(data.pop("meta_json"))
    return data


def shape_config(meta: dict, name: str) -> SimpleNamespace:
    s = meta["shapes"][name]
    return SimpleNamespace(linear_attn_config=dict(s["linear_attn"]), hidden_size=s["hidden_size"],
                           l2norm_eps=s["l2norm_eps"], rms_norm_eps=s["rms_norm_eps"])


def shape_params(data: dict, name: str) -> dict:
    pre = f"{name}.param."
    return {k[len(pre):]: v for k, v in data.items() if k.startswith(pre)}


def state_of(data: dict, key: str) -> dict:
    """{"conv": {q, k, v}, "recurrent"} saved under ``key``."""
    return {"conv": {n: data[f"{key}.conv.{n}"] for n in ("q", "k", "v")},
            "recurrent": data[f"{key}.recurrent"]}
