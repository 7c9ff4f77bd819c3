"""Globals and instruction set of the dense (Llama) VM.

Counterpart of ``megakernels/demos/latency/instructions.py:1-200``.  Opcode
ids and field order (hence the serialised words) are the reference's:

  1 LayerNorm_QKV_MatVecRopeAppend [1, layer, start_block, end_block]
  2 PartialAttention               [2, layer, kv_head, num_partials, partial_idx]
  3 AttentionReduction             [3, layer, head_start, num_partials, is_terminal, n, list..., out_idx]
  4 O_ProjResidual                 [4, layer, start_block, end_block, reduction_block]
  5 LayerNormDoubleMatVecSiLU      [5, layer, n, block...]
  6 DownProjResidual               [6, layer, start_block, end_block, reduction_block]
  7 RMS_LM_Head                    [7, start_block, end_block]
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

from torch import Tensor

from ..instructions import BaseGlobals, Instruction, serialize_reduction


@dataclass
class Globals(BaseGlobals):
    # activation buffers
    post_ln_rope_q: Tensor
    attn_out: Tensor
    attn_lse_intermediates: Tensor
    attn_out_intermediates: Tensor
    silu_out: Tensor
    logits: Tensor

    skip_attn_reduction: bool

    # block size constants
    up_gate_proj_block_size: int
    down_proj_block_size: int
    o_proj_block_size: int
    lm_head_block_size: int
    matvec_reduction_size: int
    qkv_block_size: int
    attn_kv_block_size: int
    attn_reduction_size: int


@dataclass
class LayerNorm_QKV_MatVecRopeAppend(Instruction):
    """RMSNorm + QKV matvec + RoPE on q and k + K/V append."""

    layer_idx: int
    start_output_block_idx: int
    end_output_block_idx: int

    @classmethod
    def opcode(cls) -> int:
        return 1

    @classmethod
    def prev_opcode(cls) -> int:
        return DownProjResidual.opcode()

    def block_indices(self):
        return list(range(self.start_output_block_idx, self.end_output_block_idx))

    def cost(self, globs: Globals):
        return (self.end_output_block_idx - self.start_output_block_idx) * globs.qkv_block_size * globs.hidden_size


@dataclass
class PartialAttention(Instruction):
    layer_idx: int
    kv_head_idx: int
    num_partials: int
    partial_idx: int

    @classmethod
    def opcode(cls) -> int:
        return 2

    @classmethod
    def prev_opcode(cls) -> int:
        return LayerNorm_QKV_MatVecRopeAppend.opcode()

    def cost(self, globs: Globals):
        return (globs.pos_id + 1) / self.num_partials * globs.head_dim * 2


@dataclass
class AttentionReduction(Instruction):
    layer_idx: int
    head_start_idx: int
    num_partials: int
    is_terminal: bool
    reduction_list: list[int]
    output_partial_idx: Optional[int] = None

    @classmethod
    def opcode(cls) -> int:
        return 3

    @classmethod
    def prev_opcode(cls) -> int:
        return PartialAttention.opcode()

    def cost(self, globs: Globals):
        return globs.num_attention_heads // globs.num_kv_heads * self.num_partials * globs.head_dim

    def serialize(self) -> list[int]:
        return serialize_reduction(self)


@dataclass
class MatVecAdd(Instruction):
    layer_idx: int
    start_block_idx: int
    end_block_idx: int
    reduction_block_idx: int


@dataclass
class O_ProjResidual(MatVecAdd):
    @classmethod
    def opcode(cls) -> int:
        return 4

    @classmethod
    def prev_opcode(cls) -> int:
        return AttentionReduction.opcode()

    def cost(self, globs: Globals):
        return (self.end_block_idx - self.start_block_idx) * globs.o_proj_block_size * globs.hidden_size


@dataclass
class LayerNormDoubleMatVecSiLU(Instruction):
    """RMSNorm + up and gate matvecs + SiLU over a list of row blocks."""

    layer_idx: int
    block_idxs: list[int]

    @classmethod
    def opcode(cls) -> int:
        return 5

    @classmethod
    def prev_opcode(cls) -> int:
        return O_ProjResidual.opcode()

    def cost(self, globs: Globals):
        return len(self.block_idxs) * globs.up_gate_proj_block_size * globs.hidden_size * 2


@dataclass
class DownProjResidual(MatVecAdd):
    @classmethod
    def opcode(cls) -> int:
        return 6

    @classmethod
    def prev_opcode(cls) -> int:
        return LayerNormDoubleMatVecSiLU.opcode()

    def cost(self, globs: Globals):
        return (self.end_block_idx - self.start_block_idx) * globs.down_proj_block_size * globs.hidden_size


@dataclass
class RMS_LM_Head(Instruction):
    start_output_block_idx: int
    end_output_block_idx: int

    @classmethod
    def opcode(cls) -> int:
        return 7

    @classmethod
    def prev_opcode(cls) -> int:
        return DownProjResidual.opcode()

    def cost(self, globs: Globals):
        return (self.end_output_block_idx - self.start_output_block_idx) * globs.lm_head_block_size * globs.hidden_size
