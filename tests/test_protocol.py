"""The kernel's dependency protocol, emulated on the CPU
(megakernels_amd/protocol.py): final barrier counts, deadlock-freedom of the
assignment strategies, and the failure reports the kernel would write
(time-out, unsupported opcode, bad operand) -- all forced from the host."""

import numpy as np
import pytest

from megakernels_amd.mixtral.instructions import ExpertDownProjFused, Mixtral_QKV, RmsRouterUpgate, SpeculativeExpertPredict
from megakernels_amd.mixtral.scheduler import make_globals, make_moe_dag, prefill_oproj_barrier
from megakernels_amd.mixtral.synthetic import SMALL, make_residuals, make_synthetic_mixtral, with_layers
from megakernels_amd.protocol import (
    MK_ERR_BAD_INSTRUCTION,
    MK_ERR_BAD_OPCODE,
    MK_ERR_TIMEOUT,
    MK_ERR_UNSUPPORTED_OPCODE,
    ProtocolDims,
    ProtocolError,
    simulate,
)
from megakernels_amd.scheduler import Schedule, assign_to_sms, tensorize_instructions
from oracle import python_vm as oracle


def _globs(workers=16, layers=1, **kw):
    model = make_synthetic_mixtral(with_layers(SMALL, layers), "cpu", 0)
    return model, make_globals(model, sm_count=workers, **kw)


@pytest.mark.parametrize("mode", ["rr", "zz", "wave", "dag"])
@pytest.mark.parametrize("workers", [1, 3, 16, 256])
def test_moe_schedules_complete(mode, workers):
    _, g = _globs(workers)
    sched = Schedule(g, *make_moe_dag(g, predict=True))
    tensorize_instructions(g, assign_to_sms(mode, schedule=sched))
    prefill_oproj_barrier(g)
    bar = simulate(g.instructions, g.barriers, ProtocolDims.from_globals(g))
    assert bar[0, 3, 0] == g.hidden_size // g.o_proj_block_size
    assert bar[0, 4, 0] == g.intermediate_size // g.expert_proj_block_size
    assert bar[0, 5, 0] == 2 * (g.hidden_size // g.down_proj_block_size)
    assert bar[0, 7, 0] == 1


def test_simulated_barriers_equal_oracle_pyvm():
    _, g = _globs(7, expert_proj_block_size=8, down_proj_block_size=4)
    sched = Schedule(g, *make_moe_dag(g, predict=True))
    tensorize_instructions(g, assign_to_sms("rr", schedule=sched))
    prefill_oproj_barrier(g)
    bar = simulate(g.instructions, g.barriers, ProtocolDims.from_globals(g))
    g.hidden_states.copy_(make_residuals(1, SMALL.hidden_size, seed=4)[0])
    oracle.interpret_with_pyvm(g, sched.get_linear_instructions())
    assert np.array_equal(bar, g.barriers.numpy())


def test_missing_producer_times_out():
    _, g = _globs(4)
    tensorize_instructions(g, [[], [ExpertDownProjFused(0, 0, 4, 0)], [], []])
    prefill_oproj_barrier(g)
    with pytest.raises(ProtocolError) as ei:
        simulate(g.instructions, g.barriers, ProtocolDims.from_globals(g))
    e = ei.value
    assert (e.code, e.worker, e.slot, e.opcode, e.layer) == (MK_ERR_TIMEOUT, 1, 0, 6, 0)
    assert e.expected == g.intermediate_size // g.expert_proj_block_size and e.seen == 0


def test_opcode5_waits_for_oproj():
    _, g = _globs(2)
    tensorize_instructions(g, [[RmsRouterUpgate(0, 0, 4)], []])  # no O-proj pre-fill
    with pytest.raises(ProtocolError) as ei:
        simulate(g.instructions, g.barriers, ProtocolDims.from_globals(g))
    assert ei.value.code == MK_ERR_TIMEOUT and ei.value.opcode == 5


def test_predict_chain_across_layers():
    _, g = _globs(4, layers=2)
    # layer 1's prediction waits for layer 0's down projection
    blocks5 = g.intermediate_size // g.expert_proj_block_size
    blocks6 = g.hidden_size // g.down_proj_block_size
    queues = [[SpeculativeExpertPredict(1)], [RmsRouterUpgate(0, 0, blocks5)], [ExpertDownProjFused(0, 0, blocks6, 0)], []]
    tensorize_instructions(g, queues)
    prefill_oproj_barrier(g, 0)
    bar = simulate(g.instructions, g.barriers, ProtocolDims.from_globals(g))
    assert bar[1, 7, 0] == 1 and bar[0, 5, 0] == 2 * blocks6
    tensorize_instructions(g, [[SpeculativeExpertPredict(1)], [], [], []])
    with pytest.raises(ProtocolError) as ei:
        simulate(g.instructions, g.barriers, ProtocolDims.from_globals(g))
    assert ei.value.opcode == 8 and ei.value.layer == 0


def test_unsupported_and_bad_instructions():
    _, g = _globs(2)
    dims = ProtocolDims.from_globals(g)
    tensorize_instructions(g, [[Mixtral_QKV(0, 0, 1)], []])
    with pytest.raises(ProtocolError) as ei:
        simulate(g.instructions, g.barriers, dims)
    assert ei.value.code == MK_ERR_UNSUPPORTED_OPCODE and ei.value.opcode == 1
    tensorize_instructions(g, [[ExpertDownProjFused(0, 0, 1, 1)], []])  # partial reduction unsupported
    with pytest.raises(ProtocolError) as ei:
        simulate(g.instructions, g.barriers, dims)
    assert ei.value.code == MK_ERR_BAD_INSTRUCTION
    ins = g.instructions.clone()
    ins[0, 0, 0] = 42
    with pytest.raises(ProtocolError) as ei:
        simulate(ins, g.barriers, dims)
    assert ei.value.code == MK_ERR_BAD_OPCODE
