"""Globals construction and instruction scheduling for Mixtral decode.

Counterpart of ``megakernels/mixtral/scheduler.py:24-432``:

* ``make_globals`` allocates the reference's buffers with the same shapes and
  dtypes (``:35-152``): barriers ``[L, 10, max(Hq + 2*Hkv, E)]`` int32,
  ``expert_silu_out [E, F]``, ``router_normed_hidden [H]``, selected/predicted
  indices ``[k]`` int32, selected scores ``[k]`` bf16, attention
  intermediates sized by the worker count.
* the per-opcode partitioners split output blocks over ``min(W, blocks)``
  workers with Python's ``round`` (banker's rounding), exactly as
  ``:176-232`` do, so block boundaries match the reference for equal block
  sizes.
* ``make_dag`` builds the reference's per-layer DAG (``:261-418``).

Differences, all MI355X-motivated and recorded here:

* ``expert_proj_block_size`` / ``down_proj_block_size`` default to a value
  picked for the worker count (``pick_block_size``) instead of a fixed 16:
  with 256 compute units, F = 14336 splits into 1792 blocks of 8 rows, i.e.
  exactly 7 blocks per worker, where 16-row blocks leave a 4-vs-3 imbalance.
  Passing ``16`` reproduces the reference partition.  The oracle reads the
  block sizes from the globals, so results do not depend on this choice.
* the split-KV partition count defaults to the MI355X policy of
  :func:`pick_num_attention_partitions` (chunks of >= 112 positions, up to
  min(W / kv_heads, 64) partitions per KV head) instead of the reference's (>= 256 positions, at
  most 160 / kv_heads): the kernel's partial attention is VALU-bound per
  workgroup, so more, shorter partitions finish sooner.
  ``attention_partitions="reference"`` reproduces the reference partition.
* ``qkv_block_size`` is picked the same way among 16 and 8 rows (at config
  4 and 256 workers, 8-row blocks give every worker 24 QKV rows where 16-row
  blocks leave 32 on half of them; 4-row blocks measured slower); it stays a
  divisor of head_dim.
* ``moe_overlap=True`` (off by default) partitions opcode 5 into one
  instruction per block, interleaved across workers, and launches with the
  kernel's opcode-5/6 overlap (opcode 6 starts on column chunks of the SiLU
  output as they complete instead of after the layer's last opcode-5 block).
  Indices, scores and barrier counts are unchanged; hidden states differ
  only in the fp32 summation order of the down-projection rows.
* ``make_moe_dag`` builds the MoE-only slice of one layer (optional opcode 8,
  then opcode 5 and opcode 6) for running the hot path in isolation; the
  attention prefix it skips is represented by pre-filling the O-proj barrier
  (``prefill_oproj_barrier``), the reference's ``barrier_fill`` idiom scoped
  to the one counter opcode 5 waits on.
"""

from __future__ import annotations

import math

import torch

from ..instructions import NoOp
from ..scheduler import DAG_Node, ScheduleBuilder
from ..utils import assert_div, get_sm_count
from .instructions import (
    ExpertDownProjFused,
    Mixtral_AttnReduction,
    Mixtral_OProj,
    Mixtral_PartialAttn,
    Mixtral_QKV,
    Mixtral_RMS_LM_Head,
    MixtralGlobals,
    RmsRouterUpgate,
    SpeculativeExpertPredict,
)

#: number of opcode rows in the barrier tensor (mkm/scheduler.py:61-68)
BARRIER_OPS = 10
#: reference cap on attention partitions per layer (mkm/scheduler.py:21)
ATTN_PARTITION_CAP = 160
#: partials a terminal reduction can list: its 32-word instruction holds 7
#: other words (the reference's partition policies stay within it)
MAX_REDUCTION_LIST = 25
#: partitions per KV head of the MI355X policy: a terminal reduction over
#: more than MAX_REDUCTION_LIST partials is encoded as a range (one lane per
#: partial in the kernel's reduction: 64 at most)
MAX_PARTITIONS = 64
#: fewest positions per partition of the MI355X policy (swept at config 3:
#: 17-19 partitions of 112-128 positions beat 22 of 96 by 1.5 %, and 13-15 by
#: 2 %; configs 4 and 5 stay at the cap)
MIN_PARTITION_POSITIONS = 112


def pick_num_attention_partitions(prompt_len: int, ntok: int, num_kv_heads: int, sm_count: int,
                                  policy: str = "reference", kv_block_size: int = 16) -> int:
    """Split-KV partition count.

    ``"reference"`` (mkm/scheduler.py:24-32): chunks of at least 256
    positions, at most ``min(W, 160) // kv_heads`` partitions.

    ``"mi355x"``: chunks of at least 112 positions and at most ``min(W //
    kv_heads - 1, 64)`` partitions (one worker per KV head is left for its
    reduction), trimmed so that none is empty.  A
    workgroup's partial attention is bound by how fast it pulls its K/V rows
    (and, for short partitions, by its fixed merge-and-store cost), not by
    the HBM bandwidth of the whole chip, so on 256 compute units it pays to
    spread the cache over all of them.  More than 25 partials (what one
    reduction instruction lists) are reduced through a range-encoded list
    (``Mixtral_AttnReduction.serialize``).  ``"mi355x:N"`` caps the count at
    N instead.
    """
    seq = prompt_len + ntok
    if policy == "reference":
        chunks = math.ceil(seq / 256)
        cap = min(sm_count, ATTN_PARTITION_CAP) // num_kv_heads
        return max(1, min(chunks, cap))
    cap = MAX_PARTITIONS
    if policy.startswith("mi355x:"):
        cap = int(policy.split(":", 1)[1])
        if not 1 <= cap <= MAX_PARTITIONS:
            raise ValueError(f"partition cap must be in 1..{MAX_PARTITIONS}, got {cap}")
    elif policy != "mi355x":
        raise ValueError(f"unknown partition policy {policy!r}")
    # one worker per KV head stays free of partials for its reduction, which
    # then waits while the partials run instead of starting after one
    n = max(1, min(math.ceil(seq / MIN_PARTITION_POSITIONS), sm_count // num_kv_heads - 1, cap))
    total = math.ceil(seq / kv_block_size)
    return max(1, math.ceil(total / math.ceil(total / n)))


def pick_block_size(rows: int, workers: int, candidates=(16, 8, 4)) -> int:
    """Row-block size that minimises the busiest worker's row count when
    ``rows / block`` blocks are spread over ``workers`` (ties -> larger
    block, fewer instructions)."""
    best = None
    for bs in candidates:
        if rows % bs:
            continue
        blocks = rows // bs
        busiest = math.ceil(blocks / min(workers, blocks)) * bs
        key = (busiest, -bs)
        if best is None or key < best[0]:
            best = (key, bs)
    if best is None:
        raise ValueError(f"no block size in {candidates} divides {rows}")
    return best[1]


def make_globals(
    model,
    skip_attn_reduction: bool | None = None,
    seq_len: int = 0,
    sm_count: int | None = None,
    expert_proj_block_size: int | None = None,
    down_proj_block_size: int | None = None,
    attention_partitions: str = "mi355x",
    qkv_block_size: int | None = None,
    moe_overlap: bool = False,
    upgate_rounds: int = 3,
) -> MixtralGlobals:
    """Allocate activation buffers and wrap ``model``'s stacked weights.

    ``model`` is duck-typed like the reference's ``MixtralForCausalLM``:
    ``.config``, ``.device``, ``.dtype``, ``.stacked_params`` (``qkv_proj``,
    ``attn_ln_weight``, ``o_proj``, ``ffn_ln_weight``, ``router_weight``,
    ``expert_gate``, ``expert_up``, ``expert_down``), ``.lm_head.input_norm.
    weight``, ``.lm_head.lm_head.weight``, ``.stacked_kv_cache`` and
    ``.model.rope_cos/rope_sin``.  ``sm_count`` overrides the device query
    (needed when the globals live on the CPU).  ``attention_partitions``
    picks the split-KV partition policy of ``make_dag``
    (:func:`pick_num_attention_partitions`; ``"reference"`` reproduces the
    reference's instruction list).  ``moe_overlap`` selects the interleaved
    opcode-5 partition (:func:`schedule_rms_router_upgate`) and has
    ``interpret_with_mk`` launch with the opcode-5/6 overlap.
    """
    cfg = model.config
    device = torch.device(model.device)
    dtype = model.dtype
    sp = model.stacked_params
    workers = sm_count if sm_count is not None else get_sm_count(device)

    if skip_attn_reduction is None:
        parts = pick_num_attention_partitions(seq_len + 1, 0, cfg.num_key_value_heads, workers, attention_partitions)
        skip_attn_reduction = parts == 1

    def buf(shape, buf_dtype=dtype):
        return torch.zeros(shape, device=device, dtype=buf_dtype)

    E = cfg.num_local_experts
    H = cfg.hidden_size
    F = cfg.intermediate_size
    head_dim = H // cfg.num_attention_heads
    bar_width = max(cfg.num_attention_heads + 2 * cfg.num_key_value_heads, E)
    if expert_proj_block_size is None:
        expert_proj_block_size = pick_block_size(F, workers)
    if down_proj_block_size is None:
        down_proj_block_size = pick_block_size(H, workers)
    empty = torch.empty(0, device=device, dtype=dtype)

    globs = MixtralGlobals(
        qkv_proj_weights=sp.qkv_proj,
        attn_ln_weights=sp.attn_ln_weight,
        o_proj_weights=sp.o_proj,
        mlp_ln_weights=empty,
        up_proj_weights=empty,
        gate_proj_weights=empty,
        down_proj_weights=empty,
        lm_head_norm_weights=model.lm_head.input_norm.weight,
        lm_head_weights=model.lm_head.lm_head.weight,
        k_cache=model.stacked_kv_cache[0],
        v_cache=model.stacked_kv_cache[1],
        rope_cos=model.model.rope_cos,
        rope_sin=model.model.rope_sin,
        num_hidden_layers=cfg.num_hidden_layers,
        num_attention_heads=cfg.num_attention_heads,
        num_kv_heads=cfg.num_key_value_heads,
        head_dim=head_dim,
        hidden_size=H,
        intermediate_size=F,
        vocab_size=cfg.vocab_size,
        attn_scale=1.0 / math.sqrt(head_dim),
        rms_norm_eps=cfg.rms_norm_eps,
        device=device,
        barriers=torch.zeros([cfg.num_hidden_layers, BARRIER_OPS, bar_width], dtype=torch.int32, device=device),
        pos_id=seq_len,
        hidden_states=buf(H),
        post_ln_rope_q=buf(H),
        attn_out=buf(H),
        attn_out_intermediates=buf([cfg.num_attention_heads, workers, head_dim], torch.float32),
        attn_lse_intermediates=buf([cfg.num_attention_heads, workers], torch.float32),
        expert_silu_out=buf([E, F]),
        router_normed_hidden=buf(H),
        logits=buf(cfg.vocab_size),
        selected_expert_indices=torch.zeros(cfg.num_experts_per_tok, dtype=torch.int32, device=device),
        selected_expert_scores=buf(cfg.num_experts_per_tok),
        predicted_expert_indices=torch.zeros(cfg.num_experts_per_tok, dtype=torch.int32, device=device),
        router_weights=sp.router_weight,
        expert_gate_weights=sp.expert_gate,
        expert_up_weights=sp.expert_up,
        expert_down_weights=sp.expert_down,
        ffn_ln_weights=sp.ffn_ln_weight,
        num_experts=E,
        num_experts_per_tok=cfg.num_experts_per_tok,
        skip_attn_reduction=skip_attn_reduction,
        expert_proj_block_size=expert_proj_block_size,
        down_proj_block_size=down_proj_block_size,
        o_proj_block_size=16,
        lm_head_block_size=16,
        matvec_reduction_size=math.gcd(F, H),
        qkv_block_size=qkv_block_size or pick_block_size(
            (cfg.num_attention_heads + 2 * cfg.num_key_value_heads) * head_dim, workers,
            tuple(b for b in (16, 8) if head_dim % b == 0)),
        attn_kv_block_size=16,
        attn_reduction_size=cfg.num_attention_heads // cfg.num_key_value_heads,
        router_bias=getattr(sp, "router_bias", None),
        predictor_weights=getattr(sp, "predictor_weight", None),
    )
    globs.sm_count_override = sm_count
    globs.attn_partition_policy = attention_partitions
    globs.moe_overlap = bool(moe_overlap)
    globs.upgate_rounds = int(upgate_rounds)
    return globs


# ---------------------------------------------------------------------------
# partitioners
# ---------------------------------------------------------------------------

def _spans(num_blocks: int, workers: int):
    """(start, end) per worker over ``min(workers, num_blocks)`` workers with
    banker's-rounded boundaries (Python ``round``)."""
    used = min(workers, num_blocks)
    per = num_blocks / used
    return [(round(i * per), round((i + 1) * per)) for i in range(used)]


def schedule_qkv(globs: MixtralGlobals, layer_idx: int):
    out_dim = (globs.num_attention_heads + 2 * globs.num_kv_heads) * globs.head_dim
    blocks = assert_div(out_dim, globs.qkv_block_size)
    return [Mixtral_QKV(layer_idx, s, e) for s, e in _spans(blocks, globs.sm_count())]


def schedule_rms_router_upgate(globs: MixtralGlobals, layer_idx: int):
    """The reference's contiguous spans (``mkm/scheduler.py:176-196``) or,
    with ``globs.moe_overlap``, one instruction per block in block order:
    assigned round-robin, worker ``w`` then holds blocks ``w, w + W, ...`` as
    consecutive queue entries (which the kernel runs as one pool), so every
    512-row column chunk of the SiLU output is finished by many workers at
    once and early in the stage, which is what lets opcode 6 start on it."""
    blocks = assert_div(globs.intermediate_size, globs.expert_proj_block_size)
    if getattr(globs, "moe_overlap", False):
        W = globs.sm_count()
        rounds = getattr(globs, "upgate_rounds", 3)
        if blocks % W or blocks // W < rounds:
            return [RmsRouterUpgate(layer_idx=layer_idx, start_block_idx=b, num_blocks=1) for b in range(blocks)]
        # `rounds` runs of contiguous blocks per worker; run r of every worker
        # covers one contiguous span of the FFN rows
        per = blocks // W
        out, first = [], 0
        for r in range(rounds):
            n = per * (r + 1) // rounds - per * r // rounds
            out += [RmsRouterUpgate(layer_idx=layer_idx, start_block_idx=first + w * n, num_blocks=n) for w in range(W)]
            first += W * n
        return out
    return [
        RmsRouterUpgate(layer_idx=layer_idx, start_block_idx=s, num_blocks=e - s)
        for s, e in _spans(blocks, globs.sm_count())
        if e > s
    ]


def schedule_expert_downproj_fused(globs: MixtralGlobals, layer_idx: int):
    blocks = assert_div(globs.hidden_size, globs.down_proj_block_size)
    return [
        ExpertDownProjFused(layer_idx=layer_idx, start_block_idx=s, end_block_idx=e, reduction_block_idx=0)
        for s, e in _spans(blocks, globs.sm_count())
    ]


def schedule_speculative_predict(globs: MixtralGlobals, layer_idx: int):
    return [SpeculativeExpertPredict(layer_idx=layer_idx)]


def schedule_lm_head(globs: MixtralGlobals):
    blocks = assert_div(globs.vocab_size, globs.lm_head_block_size)
    splits = globs.hidden_size // 2048
    spans = _spans(blocks, globs.sm_count())
    return [Mixtral_RMS_LM_Head(s, e, r) for r in range(splits) for s, e in spans]


# ---------------------------------------------------------------------------
# DAGs
# ---------------------------------------------------------------------------

def make_dag(globs: MixtralGlobals, stop_after_op: str | None = None, layer_limit: int | None = None,
             predict: bool = True):
    """Whole-model DAG with the reference's node order and dependencies.
    ``predict=False`` leaves out opcode 8 (the speculative expert
    prediction), which also turns off the early expert-weight loads that
    consume it: the "predictor disabled" side of BASELINE config 5."""
    nodes: list[DAG_Node] = []
    layers = layer_limit if layer_limit is not None else globs.num_hidden_layers
    last: list[DAG_Node] = []
    for layer in range(layers):
        new, last = make_dag_layer(globs, layer, last, stop_after_op, predict)
        nodes.extend(new)
    if layers == globs.num_hidden_layers and stop_after_op is None:
        head = [DAG_Node(ins, last) for ins in schedule_lm_head(globs)]
        nodes.extend(head)
        last = head
    return nodes, DAG_Node(NoOp(), last)


def make_dag_layer(globs: MixtralGlobals, layer_idx: int, prev_layer_outputs, stop_after_op: str | None = None,
                   predict: bool = True):
    parts = pick_num_attention_partitions(globs.pos_id + 1, 0, globs.num_kv_heads, globs.sm_count(),
                                          getattr(globs, "attn_partition_policy", "reference"),
                                          globs.attn_kv_block_size)
    globs.skip_attn_reduction = parts == 1
    nodes: list[DAG_Node] = []

    qkv_nodes = [DAG_Node(ins, prev_layer_outputs) for ins in schedule_qkv(globs, layer_idx)]
    by_block = {}
    for n in qkv_nodes:
        for b in n.instruction.block_indices():
            by_block[b] = n
    nodes.extend(qkv_nodes)
    if predict:
        nodes.extend(DAG_Node(ins, prev_layer_outputs) for ins in schedule_speculative_predict(globs, layer_idx))
    if stop_after_op == "qkv":
        return nodes, qkv_nodes

    bph = globs.head_dim // globs.qkv_block_size
    partial_nodes = []
    for kv in range(globs.num_kv_heads):
        k0 = (globs.num_attention_heads + kv) * globs.head_dim // globs.qkv_block_size
        v0 = (globs.num_attention_heads + globs.num_kv_heads + kv) * globs.head_dim // globs.qkv_block_size
        deps = {id(by_block[b]): by_block[b] for b in [*range(k0, k0 + bph), *range(v0, v0 + bph)]}
        for p in range(parts):
            partial_nodes.append(DAG_Node(Mixtral_PartialAttn(layer_idx, kv, parts, p), list(deps.values())))
    nodes.extend(partial_nodes)
    if stop_after_op == "partial":
        return nodes, partial_nodes

    gqa = globs.num_attention_heads // globs.num_kv_heads
    if parts > 1:
        red_nodes = []
        for kv in range(globs.num_kv_heads):
            ins = Mixtral_AttnReduction(layer_idx, kv * gqa, parts, True, list(range(parts)), None)
            red_nodes.append(DAG_Node(ins, [n for n in partial_nodes if n.instruction.kv_head_idx == kv]))
        nodes.extend(red_nodes)
        oproj_deps = red_nodes
    else:
        oproj_deps = partial_nodes
    if stop_after_op == "reduction":
        return nodes, oproj_deps

    oproj_nodes = [
        DAG_Node(Mixtral_OProj(layer_idx, b, b + 1, 0), oproj_deps)
        for b in range(assert_div(globs.hidden_size, globs.o_proj_block_size))
    ]
    nodes.extend(oproj_nodes)
    if stop_after_op == "oproj":
        return nodes, oproj_nodes

    rru_nodes = [DAG_Node(ins, oproj_nodes) for ins in schedule_rms_router_upgate(globs, layer_idx)]
    nodes.extend(rru_nodes)
    if stop_after_op in ("router", "expert_upgate", "rms_router_upgate"):
        return nodes, rru_nodes

    down_nodes = [DAG_Node(ins, rru_nodes) for ins in schedule_expert_downproj_fused(globs, layer_idx)]
    nodes.extend(down_nodes)
    if stop_after_op in (None, "downproj", "expert_downproj", "downproj_fused"):
        return nodes, down_nodes
    raise ValueError(f"unknown stop_after_op {stop_after_op!r}")


def make_moe_dag(globs: MixtralGlobals, layer_idx: int = 0, predict: bool = False,
                 stop_after_op: str | None = None):
    """MoE-only slice of one layer: [opcode 8], opcode 5 x N, opcode 6 x M.

    ``stop_after_op="rms_router_upgate"`` stops after opcode 5.  Pair with
    :func:`prefill_oproj_barrier` before launching.
    """
    nodes: list[DAG_Node] = []
    if predict:
        nodes.extend(DAG_Node(ins, []) for ins in schedule_speculative_predict(globs, layer_idx))
    rru = [DAG_Node(ins, []) for ins in schedule_rms_router_upgate(globs, layer_idx)]
    nodes.extend(rru)
    last = rru
    if stop_after_op not in ("router", "expert_upgate", "rms_router_upgate"):
        if stop_after_op not in (None, "downproj", "expert_downproj", "downproj_fused"):
            raise ValueError(f"unknown stop_after_op {stop_after_op!r}")
        down = [DAG_Node(ins, rru) for ins in schedule_expert_downproj_fused(globs, layer_idx)]
        nodes.extend(down)
        last = down
    return nodes, DAG_Node(NoOp(), last)


def expected_oproj_arrivals(globs: MixtralGlobals) -> int:
    """Arrivals opcode 5 waits for (mkm/python_vm.py:42-43)."""
    return globs.hidden_size // globs.o_proj_block_size


def expected_upgate_arrivals(globs: MixtralGlobals) -> int:
    """Arrivals opcode 6 waits for (mkm/python_vm.py:46-48)."""
    return globs.intermediate_size // globs.expert_proj_block_size


def expected_downproj_arrivals(globs: MixtralGlobals) -> int:
    """Arrivals the next layer waits for (mkm/python_vm.py:51-54)."""
    return globs.num_experts_per_tok * (globs.hidden_size // globs.down_proj_block_size)


def prefill_oproj_barrier(globs: MixtralGlobals, layer_idx: int = 0) -> None:
    """Mark layer ``layer_idx``'s O-projection as complete so opcode 5 runs
    without the attention prefix."""
    globs.barriers[layer_idx, Mixtral_OProj.opcode() - 1, 0] = expected_oproj_arrivals(globs)


class MixtralLatencyScheduleBuilder(ScheduleBuilder):
    @classmethod
    def make_globals(cls, model, seq_len: int = 0, **kw) -> MixtralGlobals:
        return make_globals(model, seq_len=seq_len, **kw)

    @classmethod
    def make_dag(cls, globs, stop_after_op=None, layer_limit=None):
        return make_dag(globs, stop_after_op, layer_limit)


class MixtralMoEScheduleBuilder(ScheduleBuilder):
    """Builds the MoE-only single-layer schedule used for the hot path."""

    @classmethod
    def make_globals(cls, model, seq_len: int = 0, **kw) -> MixtralGlobals:
        return make_globals(model, seq_len=seq_len, **kw)

    @classmethod
    def make_dag(cls, globs, stop_after_op=None, layer_limit=None):
        return make_moe_dag(globs, 0, stop_after_op=stop_after_op)
