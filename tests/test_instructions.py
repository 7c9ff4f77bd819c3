"""Instruction serialisation, queue tensorisation, assignment strategies and
partitioners -- the host half of the drop-in surface.  Expected words and
boundaries are worked out by hand from the reference's rules
(megakernels/instructions.py:97-119, megakernels/scheduler.py:155-309,
megakernels/mixtral/scheduler.py:176-232)."""

import pytest
import torch

from megakernels_amd.instructions import NoOp
from megakernels_amd.mixtral.instructions import (
    ExpertDownProjFused,
    Mixtral_AttnReduction,
    Mixtral_OProj,
    Mixtral_PartialAttn,
    Mixtral_QKV,
    Mixtral_RMS_LM_Head,
    RmsRouterUpgate,
    SpeculativeExpertPredict,
)
from megakernels_amd.mixtral.scheduler import (
    expected_downproj_arrivals,
    expected_oproj_arrivals,
    expected_upgate_arrivals,
    make_dag,
    make_globals,
    make_moe_dag,
    pick_block_size,
    pick_num_attention_partitions,
    schedule_expert_downproj_fused,
    schedule_rms_router_upgate,
)
from megakernels_amd.mixtral.synthetic import C1, SMALL, make_synthetic_mixtral, with_layers
from megakernels_amd.scheduler import (
    INTS_PER_INSTRUCTION,
    TIMING_SLOTS,
    Schedule,
    assign_to_sms,
    collect_into_waves,
    round_robin_assign_to_sms,
    serialize_and_pad,
    tensorize_instructions,
    zig_zag_assign_to_sms,
)


def test_opcodes():
    assert [c.opcode() for c in (NoOp, Mixtral_QKV, Mixtral_PartialAttn, Mixtral_AttnReduction, Mixtral_OProj,
                                  RmsRouterUpgate, ExpertDownProjFused, Mixtral_RMS_LM_Head,
                                  SpeculativeExpertPredict)] == [0, 1, 2, 3, 4, 5, 6, 7, 8]
    assert RmsRouterUpgate.prev_opcode() == 4
    assert ExpertDownProjFused.prev_opcode() == 5
    assert SpeculativeExpertPredict.prev_opcode() == 6


def test_serialize_words():
    assert NoOp().serialize() == [0]
    assert RmsRouterUpgate(3, 10, 7).serialize() == [5, 3, 10, 7]
    assert ExpertDownProjFused(1, 4, 9, 0).serialize() == [6, 1, 4, 9, 0]
    assert SpeculativeExpertPredict(2).serialize() == [8, 2]
    assert Mixtral_QKV(0, 5, 9).serialize() == [1, 0, 5, 9]
    # bool -> one word, list -> length then items, None -> 0
    assert Mixtral_AttnReduction(0, 4, 3, True, [0, 1, 2], None).serialize() == [3, 0, 4, 3, 1, 3, 0, 1, 2, 0]
    assert Mixtral_RMS_LM_Head(1, 2).serialize() == [7, 1, 2, 0]
    padded = serialize_and_pad(RmsRouterUpgate(3, 10, 7))
    assert len(padded) == INTS_PER_INSTRUCTION and padded[:4] == [5, 3, 10, 7] and not any(padded[4:])
    # more partials than a 32-word instruction lists: the range 0 .. n - 1 is
    # written as -n (an MI355X extension); any other long list is an error
    assert serialize_and_pad(Mixtral_AttnReduction(2, 4, 40, True, list(range(40))))[:8] == [3, 2, 4, 40, 1, -40, 0, 0]
    assert Mixtral_AttnReduction(0, 0, 25, True, list(range(25))).serialize()[5:7] == [25, 0]
    with pytest.raises(ValueError):
        serialize_and_pad(Mixtral_AttnReduction(0, 0, 40, True, list(range(1, 41))))
    # the kernel combines at most 64 partials (one lane each): 64 is written,
    # 65 fails while the schedule is built, not on the device
    assert serialize_and_pad(Mixtral_AttnReduction(0, 0, 64, True, list(range(64))))[5] == -64
    with pytest.raises(ValueError, match="at most 64"):
        serialize_and_pad(Mixtral_AttnReduction(0, 0, 80, True, list(range(80))))


def test_reference_policy_with_two_kv_heads_fails_when_tensorized():
    """The reference's partition policy allows min(W, 160) // kv_heads
    partitions (80 with two KV heads at 160+ workers); the schedule that
    needs an 80-partial reduction is refused when its instructions are
    written, before any launch."""
    from megakernels_amd.mixtral.scheduler import pick_num_attention_partitions

    n = pick_num_attention_partitions(32768, 0, 2, 256, "reference")
    assert n == 80
    with pytest.raises(ValueError, match="at most 64"):
        serialize_and_pad(Mixtral_AttnReduction(0, 0, n, True, list(range(n))))


def test_round_robin_and_zig_zag():
    ins = [RmsRouterUpgate(0, i, 1) for i in range(7)]
    rr = round_robin_assign_to_sms(ins, 3)
    assert [[x.start_block_idx for x in q] for q in rr] == [[0, 3, 6], [1, 4], [2, 5]]
    zz = zig_zag_assign_to_sms(ins, 3)
    assert [[x.start_block_idx for x in q] for q in zz] == [[0, 5, 6], [1, 4], [2, 3]]
    assert [len(w) for w in collect_into_waves([NoOp(), NoOp(), RmsRouterUpgate(0, 0, 1), NoOp()])] == [2, 1, 1]


def test_tensorize_pads_with_noops():
    model = make_synthetic_mixtral(SMALL, "cpu", 0)
    g = make_globals(model, sm_count=3)
    queues = [[RmsRouterUpgate(0, 0, 2)], [], [ExpertDownProjFused(0, 0, 1, 0), SpeculativeExpertPredict(0)]]
    t = tensorize_instructions(g, queues)
    assert t.shape == (3, 2, INTS_PER_INSTRUCTION) and t.dtype == torch.int32
    assert g.timings.shape == (3, 2, TIMING_SLOTS) and not g.timings.any()
    assert t[0, 0, :4].tolist() == [5, 0, 0, 2] and t[0, 1].abs().sum() == 0
    assert t[1].abs().sum() == 0
    assert t[2, 1, :2].tolist() == [8, 0]


def test_partitions_use_bankers_rounding():
    cfg_model = make_synthetic_mixtral(SMALL, "cpu", 0)
    g = make_globals(cfg_model, sm_count=256, expert_proj_block_size=16, down_proj_block_size=16)
    # reference partition at C2 shapes: 896 blocks over 256 workers, 3.5 per worker
    g.intermediate_size, g.hidden_size = 14336, 4096
    ins = schedule_rms_router_upgate(g, 0)
    assert len(ins) == 256
    starts = [i.start_block_idx for i in ins]
    # round(k * 3.5): 0, 4 (3.5 -> 4), 7, 10 (10.5 -> 10), 14, 18 (17.5 -> 18) ...
    assert starts[:6] == [0, 4, 7, 10, 14, 18]
    assert sum(i.num_blocks for i in ins) == 896
    assert all(a.start_block_idx + a.num_blocks == b.start_block_idx for a, b in zip(ins, ins[1:]))
    down = schedule_expert_downproj_fused(g, 0)
    assert len(down) == 256 and all(d.end_block_idx - d.start_block_idx == 1 for d in down)
    # fewer blocks than workers: one block each, min(W, blocks) instructions
    g.intermediate_size = 16 * 100
    assert len(schedule_rms_router_upgate(g, 0)) == 100


def test_interleaved_upgate_partition():
    """moe_overlap: one opcode-5 instruction per block, in block order, so a
    round-robin assignment gives worker w blocks w, w + W, ... as
    consecutive queue entries (the kernel's pool), and every 512-row column
    chunk is covered by blocks of many workers."""
    model = make_synthetic_mixtral(SMALL, "cpu", 0)
    g = make_globals(model, sm_count=256, expert_proj_block_size=8, down_proj_block_size=16, moe_overlap=True,
                     upgate_rounds=7)
    assert g.moe_overlap
    g.intermediate_size, g.hidden_size = 14336, 4096
    ins = schedule_rms_router_upgate(g, 3)
    assert len(ins) == 1792
    assert [(i.layer_idx, i.start_block_idx, i.num_blocks) for i in ins[:3]] == [(3, 0, 1), (3, 1, 1), (3, 2, 1)]
    assert [i.serialize()[:4] for i in ins[-1:]] == [[5, 3, 1791, 1]]
    queues = round_robin_assign_to_sms(ins, 256)
    assert [i.start_block_idx for i in queues[5]] == [5 + 256 * r for r in range(7)]
    # chunk 0 (FFN rows 0-511, blocks 0-63) is finished by 64 different workers
    assert len({b % 256 for b in range(64)}) == 64
    # two rounds (the default): runs of 3 then 4 contiguous blocks per worker,
    # round 0 covering blocks 0-767 and round 1 blocks 768-1791
    g.upgate_rounds = 2
    ins = schedule_rms_router_upgate(g, 0)
    assert len(ins) == 512
    queues = round_robin_assign_to_sms(ins, 256)
    assert [(i.start_block_idx, i.num_blocks) for i in queues[5]] == [(15, 3), (768 + 20, 4)]
    spans = sorted((i.start_block_idx, i.num_blocks) for i in ins)
    assert spans[0] == (0, 3) and all(a[0] + a[1] == b[0] for a, b in zip(spans, spans[1:]))
    assert spans[-1][0] + spans[-1][1] == 1792
    # blocks not a multiple of the worker count: one block per instruction
    g.intermediate_size = 3584
    g.expert_proj_block_size = 16
    assert len(schedule_rms_router_upgate(g, 0)) == 224
    # the default keeps the reference's contiguous spans
    g2 = make_globals(model, sm_count=256, expert_proj_block_size=8)
    assert not g2.moe_overlap
    g2.intermediate_size = 14336
    assert len(schedule_rms_router_upgate(g2, 0)) == 256


def test_pick_block_size():
    assert pick_block_size(14336, 256) == 8      # 1792 blocks: exactly 7 per worker
    assert pick_block_size(4096, 256) == 16      # 256 blocks: one each
    assert pick_block_size(3584, 256) == 16
    assert pick_block_size(1024, 256) == 4       # 256 blocks of 4 rows
    with pytest.raises(ValueError):
        pick_block_size(10, 4)


def test_barrier_closed_forms():
    model = make_synthetic_mixtral(SMALL, "cpu", 0)
    g = make_globals(model, sm_count=8, expert_proj_block_size=8, down_proj_block_size=4)
    assert expected_oproj_arrivals(g) == 512 // 16
    assert expected_upgate_arrivals(g) == 1024 // 8
    assert expected_downproj_arrivals(g) == 2 * (512 // 4)
    assert g.barriers.shape == (1, 10, max(8 + 2 * 2, 4))


def test_make_globals_buffers():
    model = make_synthetic_mixtral(C1, "cpu", 0)
    g = make_globals(model, sm_count=256)
    assert g.expert_silu_out.shape == (8, 3584) and g.expert_silu_out.dtype == torch.bfloat16
    assert g.selected_expert_indices.dtype == torch.int32 and g.selected_expert_scores.dtype == torch.bfloat16
    assert g.predicted_expert_indices.shape == (2,)
    assert g.attn_lse_intermediates.shape == (8, 256)
    assert g.matvec_reduction_size == 512  # gcd(3584, 1024)


def test_dag_structure():
    model = make_synthetic_mixtral(with_layers(SMALL, 2), "cpu", 0)
    g = make_globals(model, sm_count=16, seq_len=10)
    nodes, end = make_dag(g)
    ops = [n.instruction.opcode() for n in nodes]
    per_layer = len(ops) // 2
    assert ops.count(8) == 2
    # LM head: one column split per 2048 hidden units (none at H = 512)
    assert ops.count(7) == (g.hidden_size // 2048) * min(16, g.vocab_size // 16)
    assert ops.index(5) > ops.index(4)  # topological order within a layer
    parts = pick_num_attention_partitions(11, 0, 2, 16)
    assert ops.count(2) == 2 * 2 * parts
    assert per_layer > 0
    rru = [n for n in nodes if n.instruction.opcode() == 5 and n.instruction.layer_idx == 0]
    assert all(all(d.instruction.opcode() == 4 for d in n.dependencies) for n in rru)
    nodes, _ = make_dag(g, stop_after_op="rms_router_upgate", layer_limit=1)
    assert nodes[-1].instruction.opcode() == 5


def test_moe_dag():
    model = make_synthetic_mixtral(SMALL, "cpu", 0)
    g = make_globals(model, sm_count=16)
    nodes, end = make_moe_dag(g, predict=True)
    ops = [n.instruction.opcode() for n in nodes]
    assert ops[0] == 8 and set(ops[1:]) == {5, 6}
    nodes, _ = make_moe_dag(g, stop_after_op="rms_router_upgate")
    assert {n.instruction.opcode() for n in nodes} == {5}
    sched = Schedule(g, *make_moe_dag(g))
    for mode in ("rr", "zz", "wave", "dag"):
        queues = assign_to_sms(mode, schedule=sched)
        assert len(queues) == 16
        assert sorted(i.serialize() for q in queues for i in q) == sorted(
            i.serialize() for i in sched.get_linear_instructions())
