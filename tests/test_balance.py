"""Speed-weighted partitions (megakernels_amd/mixtral/balance.py): spans,
queue rebalancing, rate measurement from a timing record, and that a
rebalanced schedule gives the oracle's results and barrier totals."""

import numpy as np
import pytest
import torch

from megakernels_amd.mixtral.balance import (
    rebalance_queues,
    weighted_spans,
    weights_from_rates,
    worker_rates_from_timings,
)
from megakernels_amd.mixtral.instructions import ExpertDownProjFused, RmsRouterUpgate
from megakernels_amd.mixtral.scheduler import make_globals, make_moe_dag, prefill_oproj_barrier
from megakernels_amd.mixtral.synthetic import SMALL, make_residuals, make_synthetic_mixtral
from megakernels_amd.protocol import ProtocolDims, simulate
from megakernels_amd.scheduler import Schedule, assign_to_sms, tensorize_instructions
from oracle import python_vm as oracle


def test_weighted_spans_tile_and_follow_weights():
    rng = np.random.default_rng(0)
    for n in (1, 7, 100, 14336):
        for k in (1, 3, 256):
            w = rng.uniform(0.5, 1.5, k)
            spans = weighted_spans(n, w)
            assert spans[0][0] == 0 and spans[-1][1] == n
            assert all(a[1] == b[0] for a, b in zip(spans, spans[1:]))
            ideal = np.cumsum(w) / w.sum() * n
            ends = np.array([e for _, e in spans])
            assert np.all(np.abs(ends - ideal) <= 0.5 + 1e-9)
    assert weighted_spans(10, [1, 1, 2]) == [(0, 2), (2, 5), (5, 10)]
    with pytest.raises(ValueError):
        weighted_spans(10, [1, 0])


def _schedule(workers=16, mode="rr", predict=False, **kw):
    model = make_synthetic_mixtral(SMALL, "cpu", 0)
    g = make_globals(model, sm_count=workers, **kw)
    sched = Schedule(g, *make_moe_dag(g, predict=predict))
    return model, g, sched, assign_to_sms(mode, schedule=sched)


@pytest.mark.parametrize("mode,predict", [("rr", False), ("rr", True), ("dag", True), ("zz", False)])
def test_rebalance_keeps_cover_slots_and_barrier_totals(mode, predict):
    model, g, sched, queues = _schedule(mode=mode, predict=predict, expert_proj_block_size=1, down_proj_block_size=1)
    weights = np.where(np.arange(16) % 2, 0.9, 1.1)
    new = rebalance_queues(queues, g, weights)
    assert [len(q) for q in new] == [len(q) for q in queues]
    rows5, rows6 = [], []
    for q_old, q_new in zip(queues, new):
        for a, b in zip(q_old, q_new):
            assert a.opcode() == b.opcode()
            if isinstance(b, RmsRouterUpgate):
                rows5 += range(b.start_block_idx, b.start_block_idx + b.num_blocks)
            if isinstance(b, ExpertDownProjFused):
                rows6 += range(b.start_block_idx, b.end_block_idx)
    assert sorted(rows5) == list(range(SMALL.intermediate_size))
    assert sorted(rows6) == list(range(SMALL.hidden_size))
    # faster workers got more rows
    per_worker = np.zeros(16)
    for w, q in enumerate(new):
        for ins in q:
            if isinstance(ins, RmsRouterUpgate):
                per_worker[w] += ins.num_blocks
    assert per_worker[0::2].mean() > per_worker[1::2].mean()
    tensorize_instructions(g, new)
    prefill_oproj_barrier(g)
    bar = simulate(g.instructions, g.barriers, ProtocolDims.from_globals(g))
    assert bar[0, 4, 0] == SMALL.intermediate_size and bar[0, 5, 0] == 2 * SMALL.hidden_size


def test_rebalance_opcode5_only_leaves_opcode6():
    """opcodes=(5,): opcode-5 rows follow the weights, opcode-6 instructions
    stay exactly as scheduled."""
    model, g, sched, queues = _schedule(expert_proj_block_size=1)
    weights = np.where(np.arange(16) % 2, 0.9, 1.1)
    new = rebalance_queues(queues, g, weights, opcodes=(5,))
    for q_old, q_new in zip(queues, new):
        for a, b in zip(q_old, q_new):
            if isinstance(a, ExpertDownProjFused):
                assert a.serialize() == b.serialize()
    per_worker = np.zeros(16)
    for w, q in enumerate(new):
        for ins in q:
            if isinstance(ins, RmsRouterUpgate):
                per_worker[w] += ins.num_blocks
    assert per_worker.sum() == SMALL.intermediate_size
    assert per_worker[0::2].mean() > per_worker[1::2].mean()


def test_rebalanced_schedule_gives_identical_oracle_results():
    model, g, sched, queues = _schedule(expert_proj_block_size=1, down_proj_block_size=1)
    new = rebalance_queues(queues, g, np.linspace(0.6, 1.4, 16))
    W = len(new)
    linear_new = [new[i % W][i // W] for i in range(len(sched.get_linear_instructions()))]
    x = make_residuals(1, SMALL.hidden_size, seed=3)[0]
    outs = []
    for linear in (sched.get_linear_instructions(), linear_new):
        g.barriers.zero_()
        prefill_oproj_barrier(g)
        g.hidden_states.copy_(x)
        g.expert_silu_out.zero_()
        oracle.interpret_with_pyvm(g, linear)
        outs.append((g.hidden_states.clone(), g.expert_silu_out.clone(), g.barriers.clone()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_rebalance_rejects_bad_weights():
    _, g, _, queues = _schedule()
    with pytest.raises(ValueError):
        rebalance_queues(queues, g, np.ones(3))


def test_worker_rates_from_timings():
    W, Q = 4, 2
    ins = torch.zeros(W, Q, 32, dtype=torch.int32)
    tim = torch.zeros(W, Q, 128, dtype=torch.int32)
    for w in range(3):  # worker 3 runs no opcode 5
        ins[w, 0, :4] = torch.tensor([5, 0, 10 * w, 10 + w])
        tim[w, 0, 48] = 1000
        tim[w, 0, 47] = 1000 + 100 * (w + 1) * 10  # (w + 1) * 10 us
    ins[3, 1, :5] = torch.tensor([6, 0, 0, 4, 0])
    r = worker_rates_from_timings(tim, ins, expert_proj_block_size=2)
    assert np.allclose(r[:3], [2 * 10 / 10, 2 * 11 / 20, 2 * 12 / 30])
    assert np.isnan(r[3])
    # wrap-around of the 32-bit clock
    tim[0, 0, 48] = -100
    tim[0, 0, 47] = 900
    assert np.isclose(worker_rates_from_timings(tim, ins, 2)[0], 20 / 10)


def test_weights_from_rates():
    r = np.array([2.0, 1.0] * 8)
    w = weights_from_rates(r, xcds=8)
    assert np.isclose(w.mean(), 1.0)
    assert np.allclose(w[0::2] / w[1::2], 2.0)
    r2 = r.copy()
    r2[3] = np.nan  # missing measurement -> its XCD's mean
    w2 = weights_from_rates(r2, xcds=8)
    assert np.isclose(w2[3], w2[11])
