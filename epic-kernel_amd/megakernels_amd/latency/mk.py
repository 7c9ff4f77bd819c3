"""Launch the dense (Llama) VM from a latency ``Globals``.

Counterpart of ``megakernels/demos/latency/mk.py:11-68``: the KV cache is
flattened ``[L, B, T, Hkv, D] -> [(L B), T, Hkv, D]`` and ``mk_func`` is called
with the reference's 27 positional arguments on the current stream.  The
block sizes and ``matvec_reduction_size``, which the reference compiles into
its kernel, travel as keyword arguments.
"""

from __future__ import annotations

import sys
from pathlib import Path

import torch

from .instructions import Globals

PACKAGE_DIR = Path(__file__).resolve().parents[2]


def interpret_with_mk(globs: Globals, mk_func, **launch_kwargs):
    if globs.instructions is None or globs.timings is None:
        raise ValueError("call tensorize_instructions(globs, queues) before launching")
    k_cache, v_cache = globs.k_cache, globs.v_cache
    if k_cache.dim() == 5:
        k_cache, v_cache = k_cache.flatten(0, 1), v_cache.flatten(0, 1)
    kwargs = dict(
        up_gate_proj_block_size=globs.up_gate_proj_block_size,
        down_proj_block_size=globs.down_proj_block_size,
        o_proj_block_size=globs.o_proj_block_size,
        qkv_block_size=globs.qkv_block_size,
        attn_kv_block_size=globs.attn_kv_block_size,
        lm_head_block_size=globs.lm_head_block_size,
        matvec_reduction_size=globs.matvec_reduction_size,
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
        globs.mlp_ln_weights,
        globs.up_proj_weights,
        globs.gate_proj_weights,
        globs.down_proj_weights,
        globs.lm_head_norm_weights.data,
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
        globs.silu_out,
        globs.logits,
        globs.pos_id,
        globs.attn_scale,
        globs.rms_norm_eps,
        globs.skip_attn_reduction,
        **kwargs,
    )


def load_mk_func(mk_dir: Path | str | None = None):
    """Import ``mk_llama`` from ``mk_dir`` the way the reference imports its
    compiled module (``megakernels/demos/latency/mk.py:50-63``)."""
    path = str(Path(mk_dir if mk_dir is not None else PACKAGE_DIR).expanduser().absolute())
    if path not in sys.path:
        sys.path.append(path)
    from mk_llama import mk_llama  # noqa: E402

    return mk_llama


class LatencyMK_Interpreter:
    def __init__(self, mk_dir: Path | str | None = None):
        self.mk_func = load_mk_func(mk_dir)

    def interpret(self, globs: Globals, **launch_kwargs):
        return interpret_with_mk(globs, self.mk_func, **launch_kwargs)


Latency3B_MK_Interpreter = LatencyMK_Interpreter
