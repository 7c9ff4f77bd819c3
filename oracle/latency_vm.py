"""CPU oracle for the dense (Llama) VM.

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` and ``bench.py``'s
``cpu_baseline`` leg as the checker; the product path never imports it.

A restatement of ``megakernels/demos/latency/python_vm.py`` (lat/):

* ``solve_qkv``           lat/python_vm.py:162-238 (body shared with the Mixtral oracle)
* ``solve_partial_attn``  lat/python_vm.py:257-336  = the Mixtral oracle's
* ``solve_attn_reduction`` lat/python_vm.py:339-398 = the Mixtral oracle's
* ``solve_oproj``         lat/python_vm.py:96-117, over all Hq*D columns (below)
* ``solve_upgate``        lat/python_vm.py:140-178
* ``solve_downproj``      lat/python_vm.py:120-137
* ``solve_lm_head``       lat/python_vm.py:241-262

with each solver's barrier assertion and arrival.  The bf16 matvec, RMSNorm
and SiLU arithmetic is the Mixtral oracle's (``moe_oracle.c``), whose
rounding points are those of torch's bf16 CPU ops that lat/ calls.

One difference from lat/python_vm.py, on purpose: its ``o_proj_residual``
reduces over the first ``matvec_reduction_size`` columns only (``reduce=True``
with ``reduction_block_idx == 0``), which for a 3B shape (gcd(8192, 3072) =
1024 < 24 * 128) drops two thirds of ``attn_out``.  The reference's own
kernel reduces over all of them (demos/low-latency-llama/matvec_adds.cu:10-36,
REDUCTION_DIM = hidden_dim for o_proj), as does the Mixtral python_vm
(mkm/python_vm.py:203-219, reduction_size = hidden_size); so does this oracle.
"""

from __future__ import annotations

import torch

from . import python_vm as mx  # noqa: I001 (puts the package on sys.path)
from megakernels_amd.latency.instructions import (
    AttentionReduction,
    DownProjResidual,
    Globals,
    LayerNorm_QKV_MatVecRopeAppend,
    LayerNormDoubleMatVecSiLU,
    O_ProjResidual,
    PartialAttention,
    RMS_LM_Head,
)

from .python_vm import interpret_with_pyvm as _interpret
from .python_vm import matvec, rms_norm, upgate_silu


def expected_downproj_barrier(globs: Globals) -> int:
    """lat/python_vm.py:86-89: column chunks x row blocks."""
    return (globs.intermediate_size // globs.matvec_reduction_size) * (globs.hidden_size // globs.down_proj_block_size)


def expected_upgate_barrier(globs: Globals) -> int:
    return globs.intermediate_size // globs.up_gate_proj_block_size


def expected_oproj_barrier(globs: Globals) -> int:
    return globs.hidden_size // globs.o_proj_block_size


def solve_qkv(globs: Globals, ins: LayerNorm_QKV_MatVecRopeAppend):
    layer = ins.layer_idx
    if layer > 0:
        bar = globs.barriers[layer - 1, ins.prev_opcode() - 1]
        assert bar[0] == expected_downproj_barrier(globs), f"QKV layer {layer}: downproj barrier {int(bar[0])}"
    mx.qkv_rope_append(globs, ins)


def solve_upgate(globs: Globals, ins: LayerNormDoubleMatVecSiLU):
    """RMSNorm with the MLP norm, then for each listed block
    ``silu_out[rows] = bf16(bf16(silu(g)) * u)`` with bf16 g, u; one arrival
    per block."""
    layer = ins.layer_idx
    assert globs.barriers[layer, ins.prev_opcode() - 1, 0] == expected_oproj_barrier(globs)
    post_ln = rms_norm(globs.hidden_states, globs.mlp_ln_weights[layer], globs.rms_norm_eps)
    bs = globs.up_gate_proj_block_size
    bars = globs.barriers[layer, ins.opcode() - 1]
    for b in ins.block_idxs:
        r0 = b * bs
        globs.silu_out[r0:r0 + bs] = upgate_silu(globs.gate_proj_weights[layer], globs.up_proj_weights[layer],
                                                 post_ln, r0, bs)
        bars[0] += 1


def solve_downproj(globs: Globals, ins: DownProjResidual):
    """``h[rows] = bf16(h[rows] + bf16(W[rows, cols] @ silu[cols]))`` for the
    instruction's row blocks and column chunk ``reduction_block_idx``."""
    layer = ins.layer_idx
    assert globs.barriers[layer, ins.prev_opcode() - 1, 0] == expected_upgate_barrier(globs)
    R = globs.matvec_reduction_size
    c0 = ins.reduction_block_idx * R
    w = globs.down_proj_weights[layer][:, c0:c0 + R]
    vec = globs.silu_out[c0:c0 + R].contiguous()
    bs = globs.down_proj_block_size
    for b in range(ins.start_block_idx, ins.end_block_idx):
        r0 = b * bs
        globs.hidden_states[r0:r0 + bs] += matvec(w, vec, r0, bs)
    globs.barriers[layer, ins.opcode() - 1, 0] += ins.end_block_idx - ins.start_block_idx


def solve_lm_head(globs: Globals, ins: RMS_LM_Head):
    """``logits[rows] = bf16(W[rows] @ rms_norm(h))`` over all hidden columns."""
    bar = globs.barriers[globs.num_hidden_layers - 1, ins.prev_opcode() - 1]
    assert bar[0] == expected_downproj_barrier(globs), f"LM head: downproj barrier {int(bar[0])}"
    post_ln = rms_norm(globs.hidden_states, globs.lm_head_norm_weights.reshape(-1).contiguous(), globs.rms_norm_eps)
    bs = globs.lm_head_block_size
    for b in range(ins.start_output_block_idx, ins.end_output_block_idx):
        r0 = b * bs
        globs.logits[r0:r0 + bs] = matvec(globs.lm_head_weights, post_ln, r0, bs)


INSTRUCTION_TO_SOLVER = {
    LayerNorm_QKV_MatVecRopeAppend: solve_qkv,
    PartialAttention: mx.solve_partial_attn,
    AttentionReduction: mx.solve_attn_reduction,
    O_ProjResidual: mx.solve_oproj,
    LayerNormDoubleMatVecSiLU: solve_upgate,
    DownProjResidual: solve_downproj,
    RMS_LM_Head: solve_lm_head,
}


def interpret_with_pyvm(globs: Globals, instructions) -> None:
    _interpret(globs, instructions, INSTRUCTION_TO_SOLVER)
