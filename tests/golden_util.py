"""Load the golden fixtures of ``tests/golden/`` and regenerate their weights
(pinned by SHA-256, see ``tests/golden/make_golden.py``)."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "golden"))

import make_golden  # noqa: E402

from megakernels_amd.mixtral.synthetic import make_synthetic_mixtral  # noqa: E402

CASE_NAMES = tuple(make_golden.CASES)


def bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).view(torch.bfloat16)


def load_case(name: str):
    """(arrays dict of torch tensors, meta dict, CPU model with the fixture's weights)."""
    data = np.load(HERE / "golden" / f"moe_{name}.npz", allow_pickle=False)
    cfg, seed, ln_std, bias, _ = make_golden.CASES[name]
    model = make_synthetic_mixtral(cfg, "cpu", seed, ln_weight_std=ln_std, router_bias=bias)
    meta = {k[5:]: data[k] for k in data.files if k.startswith("meta_")}
    digest = make_golden.weights_digest(model.stacked_params)
    if str(meta["weights_sha256"]) != digest:
        raise RuntimeError(f"golden case {name}: regenerated weights differ from the fixture's "
                           f"(torch RNG changed?); re-run tests/golden/make_golden.py")
    arrays = {
        "hidden_in": bf16(data["hidden_in"]),
        "logits": torch.from_numpy(data["logits"]),
        "indices": torch.from_numpy(data["indices"]),
        "scores": bf16(data["scores"]),
        "normed": bf16(data["normed"]),
        "silu": bf16(data["silu"]),
        "hidden_out": bf16(data["hidden_out"]),
    }
    return arrays, meta, model
