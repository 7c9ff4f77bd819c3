"""Launch the persistent HIP megakernel from a ``MixtralGlobals``.

Counterpart of ``megakernels/mixtral/mk.py:13-107``.  ``interpret_with_mk``
flattens the stacked expert and router weights to ``[L*E, ...]`` views
(depth index = ``layer * E + expert``), reshapes the LM-head norm and the KV
cache as the reference does, and calls ``mk_func`` with the reference's
positional argument order (``mx/mixtral.cu:43-93``) on the current stream.
The block sizes, which the reference compiles into its kernel, travel as
keyword arguments, together with the two optional MoE extensions.
"""

from __future__ import annotations

import sys
from pathlib import Path

import torch

from .instructions import MixtralGlobals

PACKAGE_DIR = Path(__file__).resolve().parents[2]


def _flatten_depth(t: torch.Tensor) -> torch.Tensor:
    if t.dim() < 2:
        return t
    return t.reshape(t.shape[0] * t.shape[1], *t.shape[2:]).contiguous()


def interpret_with_mk(globs: MixtralGlobals, mk_func, **launch_kwargs):
    if globs.instructions is None or globs.timings is None:
        raise ValueError("call tensorize_instructions(globs, queues) before launching")

    k_cache = globs.k_cache
    v_cache = globs.v_cache
    if k_cache.dim() == 5:  # [L, B, T, Hkv, D] -> [(L B), T, Hkv, D]
        k_cache = k_cache.flatten(0, 1)
        v_cache = v_cache.flatten(0, 1)

    kwargs = dict(
        expert_proj_block_size=globs.expert_proj_block_size,
        down_proj_block_size=globs.down_proj_block_size,
        o_proj_block_size=globs.o_proj_block_size,
        qkv_block_size=globs.qkv_block_size,
        attn_kv_block_size=globs.attn_kv_block_size,
        lm_head_block_size=globs.lm_head_block_size,
        router_bias=globs.router_bias,
        predictor_weights=None if globs.predictor_weights is None else _flatten_depth(globs.predictor_weights),
        downproj_overlap=getattr(globs, "moe_overlap", False),
        stream=(torch.cuda.current_stream(globs.hidden_states.device)
                if globs.hidden_states.device.type == "cuda" else None),
    )
    kwargs.update(launch_kwargs)

    return mk_func(
        globs.barriers,
        globs.instructions,
        globs.timings,
        globs.qkv_proj_weights,
        globs.attn_ln_weights,
        globs.o_proj_weights,
        _flatten_depth(globs.expert_gate_weights),
        _flatten_depth(globs.expert_up_weights),
        _flatten_depth(globs.expert_down_weights),
        _flatten_depth(globs.router_weights),
        globs.ffn_ln_weights,
        globs.lm_head_norm_weights.unsqueeze(0) if globs.lm_head_norm_weights.dim() == 1 else globs.lm_head_norm_weights,
        globs.lm_head_weights.data,
        k_cache,
        v_cache,
        globs.rope_cos,
        globs.rope_sin,
        globs.hidden_states,
        globs.post_ln_rope_q,
        globs.attn_out,
        globs.attn_lse_intermediates,
        globs.attn_out_intermediates,
        globs.expert_silu_out,
        globs.router_normed_hidden,
        globs.logits,
        globs.selected_expert_indices,
        globs.selected_expert_scores,
        globs.predicted_expert_indices,
        globs.pos_id,
        globs.attn_scale,
        globs.rms_norm_eps,
        globs.skip_attn_reduction,
        **kwargs,
    )


def load_mk_func(mk_dir: Path | str | None = None):
    """Import ``mk_mixtral`` from ``mk_dir`` the way the reference does
    (``mkm/mk.py:100-104``): append the directory to ``sys.path``."""
    mk_dir = Path(mk_dir) if mk_dir is not None else PACKAGE_DIR
    path = str(mk_dir.expanduser().absolute())
    if path not in sys.path:
        sys.path.append(path)
    from mk_mixtral import mk_mixtral  # noqa: E402

    return mk_mixtral


class MK_Interpreter:
    def __init__(self, mk_dir: Path | str | None = None):
        self.mk_func = load_mk_func(mk_dir)

    def interpret(self, globs):
        raise NotImplementedError


class MixtralMK_Interpreter(MK_Interpreter):
    def interpret(self, globs: MixtralGlobals, **launch_kwargs):
        return interpret_with_mk(globs, self.mk_func, **launch_kwargs)
