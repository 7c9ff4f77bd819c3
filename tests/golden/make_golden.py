"""Write the golden fixtures for the MoE hot path.

The reference ships no golden vectors for this path (its tests need a CUDA
B200 and only print diffs), so the fixtures are produced here by an
independent evaluation of the reference's Python VM semantics with torch's
own CPU kernels, call for call as ``megakernels/mixtral/python_vm.py:228-314``
and ``megakernels/demos/latency/python_vm.py:29-56`` make them:
``rms_norm`` in fp32 with the ``.to(bfloat16)`` and the bf16 weight multiply,
``router_weights.float() @ normed.float()``, ``torch.softmax`` ->
``torch.topk`` -> renormalise, bf16 ``einsum("o i, i -> o")`` matvecs,
``F.silu(gate) * up`` in bf16, and ``hidden += (score.float() * out).to(bf16)``
per expert slot.  The C oracle (``oracle/``) and the HIP kernel are both
checked against these files.

Weights are not stored: they are regenerated from the seed with
``make_synthetic_mixtral`` (torch CPU generator) and pinned by the SHA-256 of
their bytes, so a generator change fails loudly instead of silently.  Inputs
are drawn from the same seeded stream after the weights; tokens whose top-3
router logits are within 1e-3 are redrawn so the selected pair is
unambiguous.  Stored per token: the residual input, the router logits, the
selected indices and bf16 scores, the normed hidden state, the SiLU rows of
the two selected experts, and the updated residual.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT / "epic-kernel_amd"))

from megakernels_amd.mixtral.synthetic import C1, SMALL, make_residuals, make_synthetic_mixtral  # noqa: E402

CASES = {
    # name: (config, seed, ln_weight_std, router_bias, tokens)
    "small": (SMALL, 1234, 0.1, None, 16),
    "c1": (C1, 0, None, None, 8),
    "small_bias": (SMALL, 77, 0.1, [0.5, -0.25, 0.0, 1.0], 8),
}
MARGIN = 1e-3


def weights_digest(sp) -> str:
    h = hashlib.sha256()
    for t in (sp.ffn_ln_weight, sp.router_weight, sp.expert_gate, sp.expert_up, sp.expert_down):
        h.update(t.contiguous().view(torch.int16).numpy().tobytes())
    if sp.router_bias is not None:
        h.update(sp.router_bias.contiguous().numpy().tobytes())
    return h.hexdigest()


def pyvm_layer(hidden, ffn_ln, router_w, gate, up, down, eps, k, bias=None):
    """One token through the python_vm semantics, with torch CPU ops."""
    x = hidden.to(torch.float32)
    variance = x.pow(2).mean(-1, keepdim=True)
    normed = ffn_ln * (x * torch.rsqrt(variance + eps)).to(hidden.dtype)

    logits = router_w.float() @ normed.float()
    if bias is not None:
        logits = logits + bias
    probs = torch.softmax(logits, dim=-1)
    top, idx = torch.topk(probs, k)
    top = top / top.sum()
    scores = top.to(torch.bfloat16)

    silu = []
    for e in idx.tolist():
        g = torch.einsum("oi,i->o", gate[e], normed)
        u = torch.einsum("oi,i->o", up[e], normed)
        silu.append((F.silu(g) * u).to(torch.bfloat16))

    out = hidden.clone()
    for j, e in enumerate(idx.tolist()):
        d = torch.einsum("oi,i->o", down[e], silu[j])
        out += (scores[j].float() * d).to(out.dtype)
    return logits, idx.to(torch.int32), scores, normed, torch.stack(silu), out


def margins(logits: torch.Tensor):
    top = torch.sort(logits, descending=True).values
    return float(top[0] - top[1]), float(top[1] - top[2])


def make_case(name):
    cfg, seed, ln_std, bias, n = CASES[name]
    model = make_synthetic_mixtral(cfg, "cpu", seed, ln_weight_std=ln_std, router_bias=bias)
    sp = model.stacked_params
    eps = cfg.rms_norm_eps
    b = None if sp.router_bias is None else sp.router_bias[0]
    rec = {k: [] for k in ("hidden_in", "logits", "indices", "scores", "normed", "silu", "hidden_out")}
    while len(rec["hidden_in"]) < n:
        x = make_residuals(1, cfg.hidden_size, generator=model.generator)[0]
        res = pyvm_layer(x, sp.ffn_ln_weight[0], sp.router_weight[0], sp.expert_gate[0], sp.expert_up[0],
                         sp.expert_down[0], eps, cfg.num_experts_per_tok, b)
        m01, m12 = margins(res[0])
        if m01 < MARGIN or m12 < MARGIN:
            continue
        logits, idx, scores, normed, silu, out = res
        rec["hidden_in"].append(x.view(torch.int16).numpy())
        rec["logits"].append(logits.numpy())
        rec["indices"].append(idx.numpy())
        rec["scores"].append(scores.view(torch.int16).numpy())
        rec["normed"].append(normed.view(torch.int16).numpy())
        rec["silu"].append(silu.view(torch.int16).numpy())
        rec["hidden_out"].append(out.view(torch.int16).numpy())
    arrays = {k: np.stack(v) for k, v in rec.items()}
    meta = dict(
        seed=seed, hidden=cfg.hidden_size, ffn=cfg.intermediate_size, experts=cfg.num_local_experts,
        top_k=cfg.num_experts_per_tok, eps=eps, ln_weight_std=-1.0 if ln_std is None else ln_std,
        router_bias=np.array(bias if bias is not None else [], dtype=np.float32),
        weights_sha256=weights_digest(sp), torch_version=torch.__version__,
    )
    return arrays, meta


def main():
    for name in CASES:
        arrays, meta = make_case(name)
        path = HERE / f"moe_{name}.npz"
        np.savez_compressed(path, **arrays, **{f"meta_{k}": np.asarray(v) for k, v in meta.items()})
        print(f"{path.name}: {arrays['hidden_in'].shape[0]} tokens, {path.stat().st_size} bytes")


if __name__ == "__main__":
    main()
