"""Dense (Llama) VM instruction words, partitioners and DAG against the
reference's closed forms (megakernels/demos/latency/{instructions,scheduler}.py)."""

import math

import pytest
import torch

from megakernels_amd.latency.instructions import (
    AttentionReduction,
    DownProjResidual,
    LayerNorm_QKV_MatVecRopeAppend,
    LayerNormDoubleMatVecSiLU,
    O_ProjResidual,
    PartialAttention,
    RMS_LM_Head,
)
from megakernels_amd.latency.scheduler import (
    expected_downproj_arrivals,
    make_dag,
    make_globals,
    schedule_downproj,
    schedule_lm_head,
    schedule_qkv,
    schedule_upgate,
)
from megakernels_amd.latency.synthetic import C3, LLAMA_SMALL, make_synthetic_llama
from megakernels_amd.scheduler import serialize_and_pad


def test_words():
    assert LayerNorm_QKV_MatVecRopeAppend(3, 10, 12).serialize() == [1, 3, 10, 12]
    assert PartialAttention(2, 5, 9, 4).serialize() == [2, 2, 5, 9, 4]
    assert AttentionReduction(1, 6, 3, True, [0, 1, 2], None).serialize() == [3, 1, 6, 3, 1, 3, 0, 1, 2, 0]
    assert O_ProjResidual(4, 7, 8, 0).serialize() == [4, 4, 7, 8, 0]
    assert LayerNormDoubleMatVecSiLU(5, [3, 259]).serialize() == [5, 5, 2, 3, 259]
    assert DownProjResidual(6, 30, 36, 7).serialize() == [6, 6, 30, 36, 7]
    assert RMS_LM_Head(100, 131).serialize() == [7, 100, 131]
    assert len(serialize_and_pad(RMS_LM_Head(1, 2))) == 32


class _G:
    """Shape stand-in for the C3 partitioners at 256 workers."""

    def __init__(self, cfg=C3, workers=256):
        self.num_attention_heads, self.num_kv_heads = cfg.num_attention_heads, cfg.num_key_value_heads
        self.head_dim, self.hidden_size = cfg.head_dim, cfg.hidden_size
        self.intermediate_size, self.vocab_size = cfg.intermediate_size, cfg.vocab_size
        self.qkv_block_size = self.up_gate_proj_block_size = self.down_proj_block_size = 16
        self.o_proj_block_size = self.lm_head_block_size = 16
        self.matvec_reduction_size = math.gcd(cfg.intermediate_size, cfg.hidden_size)
        self._w = workers

    def sm_count(self):
        return self._w

    def num_total_heads(self):
        return self.num_attention_heads + 2 * self.num_kv_heads


def test_c3_partitions_match_the_reference_formulas():
    g = _G()
    assert g.matvec_reduction_size == 1024
    qkv = schedule_qkv(g, 0)
    blocks = (24 + 16) * 128 // 16
    per = blocks / 256
    assert [(i.start_output_block_idx, i.end_output_block_idx) for i in qkv] == \
        [(round(w * per), round((w + 1) * per)) for w in range(256)]
    up = schedule_upgate(g, 0)
    assert len(up) == 256 and up[5].block_idxs == [5, 261]
    assert sorted(b for i in up for b in i.block_idxs) == list(range(8192 // 16))
    down = schedule_downproj(g, 0)
    jobs = [(i.reduction_block_idx, b) for i in down for b in range(i.start_block_idx, i.end_block_idx)]
    assert sorted(jobs) == [(c, b) for c in range(8) for b in range(192)]
    assert all(i.end_block_idx - i.start_block_idx == 6 for i in down)
    lm = schedule_lm_head(g)
    per = (128256 // 16) / 256
    assert [(i.start_output_block_idx, i.end_output_block_idx) for i in lm] == \
        [(round(w * per), round((w + 1) * per)) for w in range(256)]


@pytest.mark.parametrize("workers", [16, 7, 64, 3, 1])
def test_downproj_jobs_cover_each_chunk_once(workers):
    g = _G(LLAMA_SMALL, workers)
    down = schedule_downproj(g, 0)
    jobs = [(i.reduction_block_idx, b) for i in down for b in range(i.start_block_idx, i.end_block_idx)]
    assert sorted(jobs) == [(c, b) for c in range(4) for b in range(1536 // 16)]
    assert len(down) <= max(workers, 4)  # at least one instruction per column chunk


def test_full_row_down_projection_defaults_at_3b():
    """The 3B shape at 256 workers: one column chunk of 8192 and 4-row
    blocks, i.e. 768 single-chunk jobs, three (12 rows, 192 KiB) per worker."""
    from megakernels_amd.latency.scheduler import default_down_block_size, default_reduction_size

    R = default_reduction_size(8192, 3072)
    bs = default_down_block_size(3072, 256, R, 8192)
    assert (R, bs) == (8192, 4)
    g = _G(C3, 256)
    g.matvec_reduction_size, g.down_proj_block_size = R, bs
    down = schedule_downproj(g, 0)
    assert len(down) == 256 and all(i.reduction_block_idx == 0 for i in down)
    assert sorted(b for i in down for b in range(i.start_block_idx, i.end_block_idx)) == list(range(768))
    assert {i.end_block_idx - i.start_block_idx for i in down} == {3}
    # narrower chunks keep the reference's 16-row blocks
    assert default_down_block_size(3072, 256, 2048, 8192) == 16


def test_make_globals_buffers():
    model = make_synthetic_llama(LLAMA_SMALL, "cpu", 0, kv_positions=64, prefill=20)
    g = make_globals(model, seq_len=20, sm_count=16)
    H, F, Hq, Hkv, D = 1536, 2048, 12, 4, 128
    assert g.barriers.shape == (2, 10, Hq + 2 * Hkv) and g.barriers.dtype == torch.int32
    assert g.silu_out.shape == (F,) and g.logits.shape == (512,)
    assert g.attn_lse_intermediates.shape == (Hq, 16) and g.attn_out_intermediates.shape == (Hq, 16, D)
    # one column chunk (full rows, single writer per residual row)
    assert g.matvec_reduction_size == F and g.attn_reduction_size == 3
    assert g.down_proj_block_size == 16  # 96 rows on each of 16 workers at any of 16, 8, 4, 2
    assert g.attn_scale == pytest.approx(1 / math.sqrt(D))
    assert g.skip_attn_reduction  # 21 positions: one partition


@pytest.mark.parametrize("policy,parts", [("reference", 2), ("mi355x", 3)])
def test_dag_structure(policy, parts):
    model = make_synthetic_llama(LLAMA_SMALL, "cpu", 0, kv_positions=400, prefill=300)
    g = make_globals(model, seq_len=300, sm_count=16, attention_partitions=policy)
    g.pos_id = 300
    nodes, end = make_dag(g)
    ops = [n.instruction.opcode() for n in nodes]
    per_layer = {op: ops.count(op) // 2 for op in range(1, 7)}
    assert per_layer[2] == 4 * parts and per_layer[3] == 4  # partitions per KV head, one reduction each
    assert per_layer[4] == 1536 // 16
    assert ops.count(7) == 16
    # every opcode-5 node depends on all O-proj nodes of its layer; opcode 6 on all opcode-5 nodes
    up0 = [n for n in nodes if n.instruction.opcode() == 5 and n.instruction.layer_idx == 0]
    assert all(len(n.dependencies) == per_layer[4] for n in up0)
    down0 = [n for n in nodes if n.instruction.opcode() == 6 and n.instruction.layer_idx == 0]
    assert all(set(map(id, n.dependencies)) == set(map(id, up0)) for n in down0)
    assert expected_downproj_arrivals(g) == (2048 // g.matvec_reduction_size) * (1536 // g.down_proj_block_size)


@pytest.mark.parametrize("seq,kv,W", [(1, 8, 256), (64, 8, 256), (65, 8, 256), (2049, 8, 256), (4097, 8, 256),
                                      (16385, 8, 256), (301, 4, 16), (1000, 2, 7)])
def test_mi355x_partition_policy(seq, kv, W):
    """At most min(W / kv - 1, 64) partitions, none empty, more than 56
    positions each on average (n = ceil(seq / 112) before the cap); the
    reference policy is unchanged; "mi355x:N" caps the count at N."""
    from megakernels_amd.mixtral.scheduler import pick_num_attention_partitions
    from oracle.python_vm import partial_token_range

    n = pick_num_attention_partitions(seq, 0, kv, W, "mi355x")
    assert 1 <= n <= max(1, min(W // kv - 1, 64))
    ranges = [partial_token_range(seq, 16, n, p) for p in range(n)]
    assert all(b > a for a, b in ranges)
    assert [t for a, b in ranges for t in range(a, b)] == list(range(seq))
    if n < min(W // kv - 1, 64):
        assert n == 1 or seq / n > 56
    for cap in (1, 8, 25, 64):
        assert pick_num_attention_partitions(seq, 0, kv, W, f"mi355x:{cap}") <= cap
    with pytest.raises(ValueError):
        pick_num_attention_partitions(seq, 0, kv, W, "mi355x:65")
    ref = pick_num_attention_partitions(seq, 0, kv, W)
    assert ref == max(1, min(math.ceil(seq / 256), min(W, 160) // kv))
