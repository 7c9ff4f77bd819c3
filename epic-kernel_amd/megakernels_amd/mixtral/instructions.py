"""Mixtral megakernel globals and instruction set.

Counterpart of ``megakernels/mixtral/instructions.py:1-297``.  Opcode ids and
field order (hence the serialised word layout) are the reference's:

  1 Mixtral_QKV              [1, layer, start_block, end_block]
  2 Mixtral_PartialAttn      [2, layer, kv_head, num_partials, partial_idx]
  3 Mixtral_AttnReduction    [3, layer, head_start, num_partials, is_terminal, n, list..., out_idx]
  4 Mixtral_OProj            [4, layer, start_block, end_block, reduction_block]
  5 RmsRouterUpgate          [5, layer, start_block, num_blocks]
  6 ExpertDownProjFused      [6, layer, start_block, end_block, reduction_block]
  7 Mixtral_RMS_LM_Head      [7, start_block, end_block, reduction_block]
  8 SpeculativeExpertPredict [8, layer]

The HIP kernel executes every opcode 0-8.  Opcodes 1-4 and 7 (attention and
LM head) need the attention tensors; a launch without them (the MoE-only
slice) rejects those opcodes with ``MK_ERR_UNSUPPORTED_OPCODE``.

Two optional fields extend ``MixtralGlobals`` beyond the reference (both
default to ``None``, which keeps the reference's semantics exactly):

* ``router_bias``        fp32 ``[num_layers, num_experts]`` added to the router
                         logits before softmax (skewed-routing benchmark);
* ``predictor_weights``  bf16 ``[num_layers, num_experts, hidden]`` used by
                         opcode 8 instead of ``router_weights`` (noisy
                         predictor benchmark).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

from torch import Tensor

from ..instructions import BaseGlobals, Instruction, serialize_reduction

OPCODE_QKV = 1
OPCODE_PARTIAL_ATTN = 2
OPCODE_ATTN_REDUCTION = 3
OPCODE_OPROJ = 4
OPCODE_RMS_ROUTER_UPGATE = 5
OPCODE_EXPERT_DOWNPROJ_FUSED = 6
OPCODE_RMS_LM_HEAD = 7
OPCODE_SPECULATIVE_EXPERT_PREDICT = 8

#: opcodes the HIP kernel implements (0 = NoOp); 1-4 and 7 need the attention tensors
KERNEL_OPCODES = frozenset(range(9))


@dataclass
class MixtralGlobals(BaseGlobals):
    # attention activations
    post_ln_rope_q: Tensor
    attn_out: Tensor
    attn_lse_intermediates: Tensor
    attn_out_intermediates: Tensor

    # MoE activations
    expert_silu_out: Tensor          # [E, F] bf16
    router_normed_hidden: Tensor     # [H] bf16
    logits: Tensor                   # [V]

    selected_expert_indices: Tensor  # [k] int32
    selected_expert_scores: Tensor   # [k] bf16
    predicted_expert_indices: Tensor  # [k] int32

    # stacked MoE weights
    router_weights: Tensor           # [L, E, H]
    expert_gate_weights: Tensor      # [L, E, F, H]
    expert_up_weights: Tensor        # [L, E, F, H]
    expert_down_weights: Tensor      # [L, E, H, F]
    ffn_ln_weights: Tensor           # [L, H]

    num_experts: int
    num_experts_per_tok: int

    skip_attn_reduction: bool

    expert_proj_block_size: int
    down_proj_block_size: int
    o_proj_block_size: int
    lm_head_block_size: int
    matvec_reduction_size: int
    qkv_block_size: int
    attn_kv_block_size: int
    attn_reduction_size: int

    # extensions (None keeps the reference's semantics)
    router_bias: Optional[Tensor] = None
    predictor_weights: Optional[Tensor] = None

    def __post_init__(self):
        super().__post_init__()


@dataclass
class Mixtral_QKV(Instruction):
    layer_idx: int
    start_output_block_idx: int
    end_output_block_idx: int

    @classmethod
    def opcode(cls) -> int:
        return OPCODE_QKV

    @classmethod
    def prev_opcode(cls) -> int:
        return OPCODE_EXPERT_DOWNPROJ_FUSED

    def block_indices(self):
        return list(range(self.start_output_block_idx, self.end_output_block_idx))

    def cost(self, globs: MixtralGlobals) -> float:
        return (self.end_output_block_idx - self.start_output_block_idx) * globs.qkv_block_size * globs.hidden_size


@dataclass
class Mixtral_PartialAttn(Instruction):
    layer_idx: int
    kv_head_idx: int
    num_partials: int
    partial_idx: int

    @classmethod
    def opcode(cls) -> int:
        return OPCODE_PARTIAL_ATTN

    @classmethod
    def prev_opcode(cls) -> int:
        return OPCODE_QKV

    def cost(self, globs: MixtralGlobals) -> float:
        return (globs.pos_id + 1) / self.num_partials * globs.head_dim * 2


@dataclass
class Mixtral_AttnReduction(Instruction):
    layer_idx: int
    head_start_idx: int
    num_partials: int
    is_terminal: bool
    reduction_list: list[int]
    output_partial_idx: Optional[int] = None

    @classmethod
    def opcode(cls) -> int:
        return OPCODE_ATTN_REDUCTION

    @classmethod
    def prev_opcode(cls) -> int:
        return OPCODE_PARTIAL_ATTN

    def cost(self, globs: MixtralGlobals) -> float:
        return globs.num_attention_heads // globs.num_kv_heads * self.num_partials * globs.head_dim

    def serialize(self) -> list[int]:
        return serialize_reduction(self)


@dataclass
class Mixtral_OProj(Instruction):
    layer_idx: int
    start_block_idx: int
    end_block_idx: int
    reduction_block_idx: int

    @classmethod
    def opcode(cls) -> int:
        return OPCODE_OPROJ

    @classmethod
    def prev_opcode(cls) -> int:
        return OPCODE_ATTN_REDUCTION

    def cost(self, globs: MixtralGlobals) -> float:
        return (self.end_block_idx - self.start_block_idx) * globs.o_proj_block_size * globs.hidden_size


@dataclass
class RmsRouterUpgate(Instruction):
    """RMSNorm + router top-k + gate/up GEMV + SiLU for the selected experts
    over rows ``[start_block_idx, start_block_idx + num_blocks) *
    expert_proj_block_size`` of the FFN dimension."""

    layer_idx: int
    start_block_idx: int
    num_blocks: int

    @classmethod
    def opcode(cls) -> int:
        return OPCODE_RMS_ROUTER_UPGATE

    @classmethod
    def prev_opcode(cls) -> int:
        return OPCODE_OPROJ

    def block_indices(self) -> list[int]:
        return list(range(self.start_block_idx, self.start_block_idx + self.num_blocks))

    def cost(self, globs: MixtralGlobals) -> float:
        return (
            globs.num_experts * globs.hidden_size
            + self.num_blocks * globs.expert_proj_block_size * globs.hidden_size * 2 * globs.num_experts_per_tok
        )


@dataclass
class ExpertDownProjFused(Instruction):
    """Down projection of both selected experts for hidden rows
    ``[start_block_idx, end_block_idx) * down_proj_block_size``, weighted by
    the router scores and added into ``hidden_states``."""

    layer_idx: int
    start_block_idx: int
    end_block_idx: int
    reduction_block_idx: int

    @classmethod
    def opcode(cls) -> int:
        return OPCODE_EXPERT_DOWNPROJ_FUSED

    @classmethod
    def prev_opcode(cls) -> int:
        return OPCODE_RMS_ROUTER_UPGATE

    def cost(self, globs: MixtralGlobals) -> float:
        return (
            (self.end_block_idx - self.start_block_idx)
            * globs.down_proj_block_size
            * globs.intermediate_size
            * globs.num_experts_per_tok
        )


@dataclass
class Mixtral_RMS_LM_Head(Instruction):
    start_output_block_idx: int
    end_output_block_idx: int
    reduction_block_idx: int = 0

    @classmethod
    def opcode(cls) -> int:
        return OPCODE_RMS_LM_HEAD

    @classmethod
    def prev_opcode(cls) -> int:
        return OPCODE_EXPERT_DOWNPROJ_FUSED

    def cost(self, globs: MixtralGlobals) -> float:
        return (self.end_output_block_idx - self.start_output_block_idx) * globs.lm_head_block_size * globs.hidden_size


@dataclass
class SpeculativeExpertPredict(Instruction):
    """Top-k expert prediction from the pre-attention residual; the result
    lets opcode 5 start loading expert weights before its router finishes."""

    layer_idx: int

    @classmethod
    def opcode(cls) -> int:
        return OPCODE_SPECULATIVE_EXPERT_PREDICT

    @classmethod
    def prev_opcode(cls) -> int:
        return OPCODE_EXPERT_DOWNPROJ_FUSED

    def cost(self, globs: MixtralGlobals) -> float:
        return globs.num_experts * globs.hidden_size
