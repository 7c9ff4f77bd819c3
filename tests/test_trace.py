"""Timing-record analysis (megakernels_amd/trace.py) on synthetic records
whose answers are known in closed form."""

import numpy as np
import pytest

from megakernels_amd.trace import (
    TimingRecord,
    barrier_waits,
    format_report,
    hbm_utilization,
    load_record,
    phase_summary,
    save_record,
)

H, F, E = 512, 1024, 8


def _record(t0=1000):
    W, Q = 2, 2
    ins = np.zeros((W, Q, 32), dtype=np.int32)
    tim = np.zeros((W, Q, 128), dtype=np.int32)
    ins[0, 0, :4] = [5, 0, 0, 4]        # 4 blocks of 8 rows
    ins[1, 0, :4] = [5, 0, 4, 4]
    ins[0, 1, :5] = [6, 0, 0, 16, 0]    # 16 blocks of 16 rows
    ins[1, 1, :5] = [6, 0, 16, 32, 0]

    def stamp(w, q, start, wait_at, wait_done, first, done, end):
        for slot, us in ((0, start), (44, wait_at), (45, wait_done), (48, first), (47, done), (4, end)):
            tim[w, q, slot] = np.uint32((t0 + int(round(us * 100))) & 0xFFFFFFFF).view(np.int32)

    stamp(0, 0, 0, 0.5, 1.5, 2, 12, 12.5)
    stamp(1, 0, 0.2, 0.7, 1.7, 2.2, 14.2, 14.5)
    stamp(0, 1, 12.5, 12.6, 15.0, 15.5, 25.5, 26)
    stamp(1, 1, 14.5, 14.6, 15.0, 15.5, 25.5, 26)
    return TimingRecord(tim, ins, H, F, E, expert_proj_block_size=8, down_proj_block_size=16)


def test_micros_relative_and_wrapping():
    rec = _record()
    t = rec.micros()
    assert t[0, 0, 0] == 0.0 and t[1, 0, 0] == pytest.approx(0.2)
    assert t[0, 1, 4] == pytest.approx(26.0)
    assert np.isnan(t[0, 0, 100])  # never written
    # the 32-bit clock wraps between the first and last stamps
    wrapped = _record(t0=0xFFFFFFFF - 500)
    assert np.allclose(np.nan_to_num(wrapped.micros()), np.nan_to_num(t))


def test_barrier_waits():
    bw = barrier_waits(_record())
    op5, op6 = bw["by_opcode"][5], bw["by_opcode"][6]
    assert op5["count"] == 2 and op5["wait_us"] == pytest.approx(2.0)
    assert op6["wait_us"] == pytest.approx(2.4 + 0.4)
    assert op5["instr_us"] == pytest.approx(12.5 + 14.3)
    assert bw["by_layer"][0][6] == pytest.approx(2.8)


def test_hbm_utilization_conserves_bytes():
    rec = _record()
    starts, gbs, frac, total = hbm_utilization(rec, bin_us=0.5, peak_gbs=1000.0)
    b5 = 2 * 2 * 32 * H * 2
    b6 = 2 * 256 * F * 2
    assert rec.streamed_bytes(0, 0) == b5 and rec.streamed_bytes(1, 1) == b6
    assert total == 2 * b5 + 2 * b6
    # integral of the binned rate equals the bytes
    assert np.sum(gbs) * 0.5 * 1e3 == pytest.approx(total, rel=1e-9)
    assert np.allclose(frac, gbs / 1000.0)
    # during 2.2 .. 12 us both opcode-5 instructions stream
    i = int(5.0 / 0.5)
    expect = (b5 / 10.0 + b5 / 12.0) / 1e3
    assert gbs[i] == pytest.approx(expect)


def test_phase_summary_and_report(tmp_path):
    rec = _record()
    ps = phase_summary(rec)
    assert ps[("RmsRouterUpgate", "first_load")][0] == pytest.approx(2.0)
    assert ps[("ExpertDownProjFused", "done")][-1] == pytest.approx(25.5)
    path = tmp_path / "rec.npz"
    save_record(path, rec)
    back = load_record(path)
    assert np.array_equal(back.timings, rec.timings) and back.down_proj_block_size == 16
    text = format_report(back)
    assert "RmsRouterUpgate" in text and "streamed" in text


@pytest.mark.parametrize("pos,nparts,kvbs", [(0, 1, 16), (4096, 17, 16), (300, 7, 16), (33, 8, 4)])
def test_partial_attention_bytes_cover_the_cache(pos, nparts, kvbs):
    """Opcode-2 byte model: the partitions of one KV head read every cached
    position once, K and V rows of head_dim bf16 each -- the same split as
    the oracle's partial_token_range."""
    from oracle import python_vm as oracle

    D = 128
    ins = np.zeros((1, nparts, 32), dtype=np.int32)
    for q in range(nparts):
        ins[0, q, :5] = [2, 0, 3, nparts, q]
    rec = TimingRecord(np.zeros((1, nparts, 128), np.int32), ins, H, F, E, 8, 16, head_dim=D, num_kv_heads=8,
                       attn_kv_block_size=kvbs, pos_id=pos)
    per = [rec.streamed_bytes(0, q) for q in range(nparts)]
    assert sum(per) == (pos + 1) * 2 * D * 2
    for q in range(nparts):
        a, b = oracle.partial_token_range(pos + 1, kvbs, nparts, q)
        assert per[q] == max(b - a, 0) * 2 * D * 2  # trailing partitions may be empty


def test_record_roundtrip_keeps_attention_fields(tmp_path):
    rec = _record()
    rec.head_dim, rec.num_kv_heads, rec.attn_kv_block_size, rec.pos_id = 128, 8, 16, 4096
    save_record(tmp_path / "r.npz", rec)
    back = load_record(tmp_path / "r.npz")
    assert (back.head_dim, back.num_kv_heads, back.attn_kv_block_size, back.pos_id) == (128, 8, 16, 4096)


@pytest.mark.parametrize("red", [512, 2048])
def test_dense_vm_byte_model_covers_each_weight_once(red):
    """For the dense (Llama) VM the per-instruction byte model adds up to
    each layer's up+gate, down and O/QKV weights, and the LM head, once
    (down projection in column chunks of 512, or full rows)."""
    from megakernels_amd.latency.scheduler import make_dag, make_globals
    from megakernels_amd.latency.synthetic import LLAMA_SMALL, make_synthetic_llama
    from megakernels_amd.scheduler import Schedule, assign_to_sms, tensorize_instructions

    model = make_synthetic_llama(LLAMA_SMALL, "cpu", 0, kv_positions=64, prefill=40)
    g = make_globals(model, seq_len=40, sm_count=16, matvec_reduction_size=red)
    g.pos_id = 40
    tensorize_instructions(g, assign_to_sms("rr", schedule=Schedule(g, *make_dag(g))))
    rec = TimingRecord.from_globals(g)
    assert rec.dense and rec.red_cols == red and rec.opcode_names[6] == "DownProjResidual"
    W, Q = rec.instructions.shape[:2]
    by_op = {}
    for w in range(W):
        for q in range(Q):
            op = int(rec.instructions[w, q, 0])
            by_op[op] = by_op.get(op, 0) + rec.streamed_bytes(w, q)
    c = LLAMA_SMALL
    L, H, F, D = c.num_hidden_layers, c.hidden_size, c.intermediate_size, c.head_dim
    assert by_op[5] == L * 2 * F * H * 2
    assert by_op[6] == L * H * F * 2
    assert by_op[7] == c.vocab_size * H * 2
    assert by_op[1] == L * (c.num_attention_heads + 2 * c.num_key_value_heads) * D * H * 2
    assert by_op[4] == L * H * c.num_attention_heads * D * 2
    assert by_op[2] == L * c.num_key_value_heads * 41 * 2 * D * 2


def test_prediction_agreement_from_the_record():
    """Slot 50 of each layer's first opcode-5 instruction holds the predicted
    and selected experts (bytes p0, p1, s0, s1)."""
    from megakernels_amd.trace import prediction_agreement

    W, Q = 1, 6
    ins = np.zeros((W, Q, 32), dtype=np.int32)
    tim = np.zeros((W, Q, 128), dtype=np.int32)
    packs = [(3, 5, 3, 5), (3, 5, 5, 3), (1, 2, 1, 7), (0xFF, 0xFF, 2, 4)]
    for q, (p0, p1, s0, s1) in enumerate(packs):
        ins[0, q, :4] = [5, q, 0, 4]
        tim[0, q, 50] = np.uint32(p0 | p1 << 8 | s0 << 16 | s1 << 24).view(np.int32)
    ins[0, 4, :4] = [5, 0, 4, 4]  # a second instruction of layer 0: ignored
    tim[0, 4, 50] = np.uint32(1 | 2 << 8 | 6 << 16 | 7 << 24).view(np.int32)
    rec = TimingRecord(tim, ins, H, F, E, 8, 16)
    n, top1, top2 = prediction_agreement(rec)
    assert n == 3  # the layer without a prediction is left out
    assert top1 == pytest.approx(2 / 3) and top2 == pytest.approx(2 / 3)
    assert "top-2 set agreement 66.7%" in format_report(rec)


def test_pooled_opcode5_slots_share_the_first_slots_window():
    """Consecutive opcode-5 instructions of one layer on one worker run as one
    item pool: the kernel stamps the first slot and copies its start, wait,
    first-load and done-store times into the pooled slots (each gets its own
    end).  Every pooled slot's bytes are then counted, spread over the same
    window, and the binned rate still integrates to the bytes."""
    W, Q, t0 = 1, 3, 5000
    ins = np.zeros((W, Q, 32), dtype=np.int32)
    tim = np.zeros((W, Q, 128), dtype=np.int32)
    ins[0, 0, :4] = [5, 0, 0, 4]  # 4 blocks of 8 rows
    ins[0, 1, :4] = [5, 0, 4, 2]  # pooled with slot 0: 2 blocks
    ins[0, 2, :5] = [6, 0, 0, 32, 0]

    def put(q, slot, us):
        tim[0, q, slot] = np.uint32((t0 + int(round(us * 100))) & 0xFFFFFFFF).view(np.int32)

    for q, end in ((0, 10.5), (1, 10.6)):
        for slot, us in ((0, 0.0), (44, 0.5), (45, 1.0), (48, 2.0), (47, 10.0)):
            put(q, slot, us)
        put(q, 4, end)
    for slot, us in ((0, 10.6), (44, 10.7), (45, 11.0), (48, 11.5), (47, 20.0), (4, 20.5)):
        put(2, slot, us)
    rec = TimingRecord(tim, ins, H, F, E, expert_proj_block_size=8, down_proj_block_size=16)
    b0, b1, b6 = rec.streamed_bytes(0, 0), rec.streamed_bytes(0, 1), rec.streamed_bytes(0, 2)
    assert b0 == 2 * 2 * 32 * H * 2 and b1 == b0 // 2
    starts, gbs, frac, total = hbm_utilization(rec, bin_us=0.5, peak_gbs=1000.0)
    assert total == b0 + b1 + b6
    assert np.sum(gbs) * 0.5 * 1e3 == pytest.approx(total, rel=1e-9)
    # inside the shared window (2 .. 10 us) both pooled slots stream
    assert gbs[int(5.0 / 0.5)] == pytest.approx((b0 + b1) / 8.0 / 1e3)
    bw = barrier_waits(rec)
    assert bw["by_opcode"][5]["count"] == 2
    assert bw["by_opcode"][5]["wait_us"] == pytest.approx(2 * 0.5)
