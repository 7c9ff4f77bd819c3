"""Globals construction and instruction scheduling for the dense (Llama) VM.

Counterpart of ``megakernels/demos/latency/scheduler.py:1-440``:

* ``make_globals`` allocates the reference's buffers with the same shapes and
  dtypes (``:39-147``): barriers ``[L, 10, Hq + 2*Hkv]`` int32, ``silu_out
  [F]``, attention intermediates sized by the worker count, block sizes 16;
  ``matvec_reduction_size`` is the whole FFN width F (one column chunk:
  every residual row has one writer, so the down projection adds in
  python_vm's order and relaunches are bit-identical;
  ``default_reduction_size``), with down-projection blocks sized to spread
  the rows evenly (``default_down_block_size``).
* the partitioners follow ``:150-264``: QKV and LM-head blocks in contiguous
  banker's-rounded spans, up/gate blocks strided by the worker count, and
  down-projection (column chunk, row block) jobs split over workers so that
  each instruction stays within one column chunk.
* ``make_dag`` builds the per-layer DAG of ``:267-428``.
* ``qkv_block_size`` is 16 rows, as in the reference: the kernel stages a
  QKV block's rows on chip before its wait, and 16-row blocks measured
  faster than the 8-row ones that balance the row count (at 3B and 256
  workers: 24 rows on every worker instead of 32 on some and 16 on others).
  The split-KV partition count follows the MI355X policy of the Mixtral
  scheduler; ``attention_partitions="reference"`` restores the reference's.

The reference asserts more than one block per worker in every partitioner
(it targets 132-160 SMs and 1B/3B shapes); here a partitioner with fewer
blocks than workers uses ``min(W, blocks)`` of them, as the Mixtral
partitioners do, so small test shapes schedule too.
"""

from __future__ import annotations

import math

import torch

from ..instructions import NoOp
from ..scheduler import DAG_Node, ScheduleBuilder
from ..utils import assert_div, get_sm_count
from ..mixtral.scheduler import pick_block_size, pick_num_attention_partitions
from .instructions import (
    AttentionReduction,
    DownProjResidual,
    Globals,
    LayerNorm_QKV_MatVecRopeAppend,
    LayerNormDoubleMatVecSiLU,
    O_ProjResidual,
    PartialAttention,
    RMS_LM_Head,
)

#: opcode rows of the barrier tensor (latency/scheduler.py:67-74)
BARRIER_OPS = 10


def default_reduction_size(intermediate: int, hidden: int) -> int:
    """Column chunk of the dense down-projection (``matvec_reduction_size``):
    the whole FFN width when it is a multiple of 512.  Each row then has a
    single writer, which adds its one bf16 partial into the residual with a
    plain read-modify-write in python_vm's order, so results are
    reproducible bit for bit.  With narrower chunks the partials of a row
    come from different workers and are added with packed bf16 atomics in
    arrival order (python_vm adds them in chunk order), which made relaunches
    of the 28-layer 3B shape drift by 4 % in the logits."""
    if intermediate % 512 == 0:
        return intermediate
    return math.gcd(intermediate, hidden)


def default_down_block_size(hidden: int, workers: int, reduction: int, intermediate: int) -> int:
    """Rows per down-projection block: with full-width rows, the size that
    leaves the busiest worker the fewest rows (3B shape, 256 workers: 4 rows,
    768 blocks, 12 rows per worker); with column chunks, the reference's 16."""
    if reduction == intermediate:
        return pick_block_size(hidden, workers, (16, 8, 4, 2))
    return 16


def make_globals(model, skip_attn_reduction: bool | None = None, seq_len: int = 0,
                 sm_count: int | None = None, attention_partitions: str = "mi355x",
                 qkv_block_size: int | None = None, **block_sizes) -> Globals:
    """Activation buffers plus ``model``'s stacked weights (duck-typed like
    the reference's ``LlamaForCausalLM``); ``sm_count`` overrides the device
    query (needed when the globals live on the CPU); ``attention_partitions``
    is the split-KV partition policy (the Mixtral scheduler's
    ``pick_num_attention_partitions``; ``"reference"`` reproduces the
    reference's instruction list).  ``block_sizes`` override the defaults of
    ``up_gate_proj_block_size``, ``down_proj_block_size``,
    ``o_proj_block_size``, ``lm_head_block_size`` and
    ``matvec_reduction_size``."""
    allowed = {"up_gate_proj_block_size", "down_proj_block_size", "o_proj_block_size", "lm_head_block_size",
               "matvec_reduction_size"}
    unknown = set(block_sizes) - allowed
    if unknown:
        raise TypeError(f"unknown block sizes {sorted(unknown)}")
    cfg = model.config
    device = torch.device(model.device)
    dtype = model.dtype
    workers = sm_count if sm_count is not None else get_sm_count(device)
    if skip_attn_reduction is None:
        parts = pick_num_attention_partitions(seq_len + 1, 0, cfg.num_key_value_heads, workers, attention_partitions)
        skip_attn_reduction = parts == 1
    sp = model.stacked_params
    Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    reduction = block_sizes.get("matvec_reduction_size",
                                default_reduction_size(cfg.intermediate_size, cfg.hidden_size))

    def buf(shape, buf_dtype=dtype):
        return torch.zeros(shape, device=device, dtype=buf_dtype)

    globs = Globals(
        qkv_proj_weights=sp.qkv_proj,
        attn_ln_weights=sp.attn_ln_weight,
        o_proj_weights=sp.o_proj,
        mlp_ln_weights=sp.mlp_ln_weight,
        up_proj_weights=sp.up_proj,
        gate_proj_weights=sp.gate_proj,
        down_proj_weights=sp.down_proj,
        lm_head_norm_weights=model.lm_head.input_norm.weight,
        lm_head_weights=model.lm_head.lm_head.weight,
        k_cache=model.stacked_kv_cache[0],
        v_cache=model.stacked_kv_cache[1],
        rope_cos=model.model.rope_cos,
        rope_sin=model.model.rope_sin,
        num_hidden_layers=cfg.num_hidden_layers,
        num_attention_heads=Hq,
        num_kv_heads=Hkv,
        head_dim=D,
        hidden_size=cfg.hidden_size,
        intermediate_size=cfg.intermediate_size,
        vocab_size=cfg.vocab_size,
        attn_scale=1 / math.sqrt(D),
        rms_norm_eps=cfg.rms_norm_eps,
        device=device,
        hidden_states=buf(cfg.hidden_size),
        barriers=torch.zeros([cfg.num_hidden_layers, BARRIER_OPS, Hq + 2 * Hkv], dtype=torch.int32, device=device),
        pos_id=seq_len,
        post_ln_rope_q=buf(Hq * D),
        attn_out=buf(Hq * D),
        attn_lse_intermediates=buf([Hq, workers], torch.float32),
        attn_out_intermediates=buf([Hq, workers, D], torch.float32),
        silu_out=buf(cfg.intermediate_size),
        logits=buf(cfg.vocab_size),
        skip_attn_reduction=skip_attn_reduction,
        up_gate_proj_block_size=block_sizes.get("up_gate_proj_block_size", 16),
        down_proj_block_size=block_sizes.get("down_proj_block_size", default_down_block_size(
            cfg.hidden_size, workers, reduction, cfg.intermediate_size)),
        o_proj_block_size=block_sizes.get("o_proj_block_size", 16),
        lm_head_block_size=block_sizes.get("lm_head_block_size", 16),
        matvec_reduction_size=reduction,
        # 16-row QKV blocks: the kernel stages a block's rows on chip before
        # its wait, so fewer, larger blocks pay (config 3: 547.3 -> 550.4
        # tokens/s against 8-row blocks)
        qkv_block_size=qkv_block_size or (16 if D % 16 == 0 else 8),
        attn_kv_block_size=16,
        attn_reduction_size=Hq // Hkv,
    )
    globs.sm_count_override = sm_count
    globs.attn_partition_policy = attention_partitions
    return globs


# ---------------------------------------------------------------------------
# partitioners
# ---------------------------------------------------------------------------

def _spans(num_blocks: int, workers: int):
    used = min(workers, num_blocks)
    per = num_blocks / used
    return [(round(i * per), round((i + 1) * per)) for i in range(used)]


def schedule_qkv(globs: Globals, layer_idx: int):
    blocks = assert_div(globs.num_total_heads() * globs.head_dim, globs.qkv_block_size)
    return [LayerNorm_QKV_MatVecRopeAppend(layer_idx, s, e) for s, e in _spans(blocks, globs.sm_count())]


def schedule_upgate(globs: Globals, layer_idx: int):
    """Blocks strided by the worker count (latency/scheduler.py:176-196)."""
    blocks = assert_div(globs.intermediate_size, globs.up_gate_proj_block_size)
    W = min(globs.sm_count(), blocks)
    return [LayerNormDoubleMatVecSiLU(layer_idx, list(range(w, blocks, W))) for w in range(W)]


def schedule_downproj(globs: Globals, layer_idx: int):
    """(column chunk, row block) jobs in chunk-major order; worker w takes
    ``round(jobs_left / workers_left)`` of them, cut at the chunk boundary
    (latency/scheduler.py:199-247).  With fewer workers than the cuts need
    (fewer workers than column chunks), the jobs a cut leaves over become
    further instructions, where the reference's loop would drop them."""
    num_down = assert_div(globs.hidden_size, globs.down_proj_block_size)
    num_cols = assert_div(globs.intermediate_size, globs.matvec_reduction_size)
    jobs = [(c, b) for c in range(num_cols) for b in range(num_down)]
    W = min(globs.sm_count(), len(jobs))
    out, done, w = [], 0, 0
    while done < len(jobs):
        left = len(jobs) - done
        take = max(1, round(left / max(1, W - w)))
        raw = jobs[done:done + take]
        col = raw[0][0]
        sliced = [j for j in raw if j[0] == col]
        start = sliced[0][1]
        out.append(DownProjResidual(layer_idx, start, start + len(sliced), col))
        done += len(sliced)
        w += 1
    return out


def schedule_lm_head(globs: Globals):
    blocks = assert_div(globs.vocab_size, globs.lm_head_block_size)
    return [RMS_LM_Head(s, e) for s, e in _spans(blocks, globs.sm_count())]


# ---------------------------------------------------------------------------
# DAG
# ---------------------------------------------------------------------------

def make_dag(globs: Globals, stop_after_op: str | None = None, layer_limit: int | None = None):
    nodes: list[DAG_Node] = []
    layers = layer_limit if layer_limit is not None else globs.num_hidden_layers
    last: list[DAG_Node] = []
    for layer in range(layers):
        new, last = make_dag_layer(globs, layer, last, stop_after_op)
        nodes.extend(new)
    if layers == globs.num_hidden_layers and stop_after_op is None:
        head = [DAG_Node(ins, last) for ins in schedule_lm_head(globs)]
        nodes.extend(head)
        last = head
    return nodes, DAG_Node(NoOp(), last)


def make_dag_layer(globs: Globals, layer_idx: int, prev_layer_outputs, stop_after_op: str | None = None):
    parts = pick_num_attention_partitions(globs.pos_id + 1, 0, globs.num_kv_heads, globs.sm_count(),
                                          getattr(globs, "attn_partition_policy", "reference"),
                                          globs.attn_kv_block_size)
    globs.skip_attn_reduction = parts == 1
    nodes: list[DAG_Node] = []

    qkv_nodes = [DAG_Node(ins, prev_layer_outputs) for ins in schedule_qkv(globs, layer_idx)]
    by_block = {b: n for n in qkv_nodes for b in n.instruction.block_indices()}
    nodes.extend(qkv_nodes)
    if stop_after_op == "qkv":
        return nodes, qkv_nodes

    bph = assert_div(globs.head_dim, globs.qkv_block_size)
    partial_nodes = []
    for kv in range(globs.num_kv_heads):
        k0 = (globs.num_attention_heads + kv) * globs.head_dim // globs.qkv_block_size
        v0 = (globs.num_attention_heads + globs.num_kv_heads + kv) * globs.head_dim // globs.qkv_block_size
        deps = {id(by_block[b]): by_block[b] for b in [*range(k0, k0 + bph), *range(v0, v0 + bph)]}
        for p in range(parts):
            partial_nodes.append(DAG_Node(PartialAttention(layer_idx, kv, parts, p), list(deps.values())))
    nodes.extend(partial_nodes)
    if stop_after_op == "partial":
        return nodes, partial_nodes

    gqa = globs.num_attention_heads // globs.num_kv_heads
    if parts > 1:
        red_nodes = []
        for kv in range(globs.num_kv_heads):
            ins = AttentionReduction(layer_idx, kv * gqa, parts, True, list(range(parts)), None)
            red_nodes.append(DAG_Node(ins, [n for n in partial_nodes if n.instruction.kv_head_idx == kv]))
        nodes.extend(red_nodes)
        oproj_deps = red_nodes
    else:
        oproj_deps = partial_nodes
    if stop_after_op == "reduction":
        return nodes, oproj_deps

    oproj_nodes = [DAG_Node(O_ProjResidual(layer_idx, b, b + 1, 0), oproj_deps)
                   for b in range(assert_div(globs.hidden_size, globs.o_proj_block_size))]
    nodes.extend(oproj_nodes)
    if stop_after_op == "oproj":
        return nodes, oproj_nodes

    upgate_nodes = [DAG_Node(ins, oproj_nodes) for ins in schedule_upgate(globs, layer_idx)]
    nodes.extend(upgate_nodes)
    if stop_after_op == "upgate":
        return nodes, upgate_nodes

    down_nodes = [DAG_Node(ins, upgate_nodes) for ins in schedule_downproj(globs, layer_idx)]
    nodes.extend(down_nodes)
    if stop_after_op in (None, "downproj"):
        return nodes, down_nodes
    raise ValueError(f"unknown stop_after_op {stop_after_op!r}")


def expected_downproj_arrivals(globs: Globals) -> int:
    """Arrivals that complete a layer (latency/python_vm.py:86-89)."""
    return (globs.intermediate_size // globs.matvec_reduction_size) * (globs.hidden_size // globs.down_proj_block_size)


class LatencyScheduleBuilder(ScheduleBuilder):
    @classmethod
    def make_globals(cls, model, seq_len: int = 0, **kw) -> Globals:
        return make_globals(model, seq_len=seq_len, **kw)

    @classmethod
    def make_dag(cls, globs, stop_after_op=None, layer_limit=None):
        return make_dag(globs, stop_after_op, layer_limit)
