"""Instruction base classes and the globals container.

Counterpart of ``megakernels/instructions.py:10-127``:

* ``BaseGlobals`` keeps the reference's field set and order (model weights,
  KV cache, RoPE tables, model constants, ``hidden_states``, ``barriers``,
  ``pos_id``) because subclasses extend it positionally.
* ``Instruction.serialize`` produces the reference's word layout: the opcode,
  then every dataclass field in declaration order (``global_idx`` skipped);
  an ``int`` (or ``bool``) is one word, a list/tuple is its length followed by
  its items, ``None`` is a single 0.  The persistent kernel decodes exactly
  this layout.
"""

from __future__ import annotations

from dataclasses import dataclass, fields
from typing import Any

from torch import Tensor

from .utils import get_sm_count


@dataclass
class BaseGlobals:
    # stacked model parameters (layer-major)
    qkv_proj_weights: Tensor
    attn_ln_weights: Tensor
    o_proj_weights: Tensor
    mlp_ln_weights: Tensor
    up_proj_weights: Tensor
    gate_proj_weights: Tensor
    down_proj_weights: Tensor
    lm_head_norm_weights: Tensor
    lm_head_weights: Tensor
    k_cache: Tensor
    v_cache: Tensor

    rope_cos: Tensor
    rope_sin: Tensor

    num_hidden_layers: int
    num_attention_heads: int
    num_kv_heads: int
    head_dim: int
    hidden_size: int
    intermediate_size: int
    vocab_size: int

    attn_scale: float
    rms_norm_eps: float
    device: Any

    hidden_states: Tensor
    barriers: Tensor

    pos_id: int

    def __post_init__(self):
        # filled in by tensorize_instructions
        self.instructions: Tensor | None = None
        self.timings: Tensor | None = None
        # Worker count used when the globals live on a device that cannot be
        # queried (CPU-side scheduling and tests).
        self.sm_count_override: int | None = None

    def sm_count(self) -> int:
        if self.sm_count_override is not None:
            return self.sm_count_override
        return get_sm_count(self.device)

    def diff(self, other: "BaseGlobals", skip_kv_cache: bool = False):
        """Print max |a-b| and mean relative difference for every activation."""
        out = {}
        for f in fields(self):
            a = getattr(self, f.name)
            if not isinstance(a, Tensor):
                continue
            if "weights" in f.name or f.name in ("rope_cos", "rope_sin"):
                continue
            if skip_kv_cache and "cache" in f.name:
                continue
            out[f.name] = diff_tensors(a, getattr(other, f.name), f.name)
        return out

    def num_total_heads(self) -> int:
        return self.num_attention_heads + 2 * self.num_kv_heads


def diff_tensors(a: Tensor, b: Tensor, name: str):
    """Same report as ``megakernels/instructions.py:72-80``: max absolute
    difference and mean symmetric relative difference (2|a-b|/(|a|+|b|+1e-6))."""
    a32 = a.detach().float().cpu()
    b32 = b.detach().float().cpu()
    diff = a32 - b32
    adiff = diff.abs()
    rdiff = 2 * adiff / (a32.abs() + b32.abs() + 1e-6)
    max_a = adiff.max().item() if adiff.numel() else 0.0
    mean_r = rdiff.mean().item() if rdiff.numel() else 0.0
    print(f"{name}: max adiff: {max_a}, mean rdiff: {mean_r}")
    return diff, adiff, rdiff


@dataclass
class Instruction:
    @classmethod
    def opcode(cls) -> int:
        raise NotImplementedError

    @classmethod
    def prev_opcode(cls) -> int:
        raise NotImplementedError

    @classmethod
    def tags(cls) -> dict[str, Any]:
        return {}

    def cost(self, globs) -> float:
        return 0.0

    def serialize(self) -> list[int]:
        words = [int(self.opcode())]
        for f in fields(self):
            if f.name == "global_idx":
                continue
            value = getattr(self, f.name)
            if value is None:
                words.append(0)
            elif isinstance(value, (bool, int)):
                words.append(int(value))
            elif isinstance(value, (list, tuple)):
                words.append(len(value))
                words.extend(int(v) for v in value)
            else:
                raise ValueError(
                    f"{type(self).__name__}.{f.name}: cannot serialise {value!r}"
                )
        return words


#: partials a reduction instruction lists explicitly: its 32-word instruction
#: holds 7 other words
MAX_LISTED_PARTIALS = 25
#: partials one reduction instruction can combine at all: the kernel reads a
#: head's partition LSEs with one wave, one lane each
MAX_REDUCED_PARTIALS = 64


def serialize_reduction(ins) -> list[int]:
    """Words of an attention-reduction instruction (opcode 3): the
    reference's layout (``[3, layer, head_start, num_partials, is_terminal,
    n, list..., output_partial_idx]``) while the list fits the 32-word
    instruction (MAX_LISTED_PARTIALS entries).  A longer list that is the
    range ``0 .. n - 1`` is written as ``-n`` with no entries (no reference
    counterpart: the MI355X partition policy splits the cache over up to 64
    partitions per KV head); any other longer list is an error, and so is a
    list of more than MAX_REDUCED_PARTIALS, which the kernel cannot reduce
    (the reference policy allows ``min(W, 160) // kv_heads`` partitions: 80
    with two KV heads)."""
    n = len(ins.reduction_list)
    if n > MAX_REDUCED_PARTIALS:
        raise ValueError(f"{type(ins).__name__}: {n} partials to reduce; one instruction combines at most "
                         f"{MAX_REDUCED_PARTIALS} (use fewer attention partitions)")
    if n > MAX_LISTED_PARTIALS and list(ins.reduction_list) == list(range(n)):
        out = 0 if ins.output_partial_idx is None else int(ins.output_partial_idx)
        return [int(ins.opcode()), int(ins.layer_idx), int(ins.head_start_idx), int(ins.num_partials),
                int(ins.is_terminal), -n, out]
    return Instruction.serialize(ins)


@dataclass
class NoOp(Instruction):
    @classmethod
    def opcode(cls) -> int:
        return 0
