"""GPU failure paths.  Every condition is forced from the host through the
kernel's own bounded checks (a tiny spin limit on a wait whose producer is
missing, an opcode the kernel does not implement, an out-of-range operand),
so every workgroup still exits normally."""

import pytest
import torch

import mk_mixtral
from megakernels_amd.mixtral.instructions import ExpertDownProjFused, Mixtral_QKV, RmsRouterUpgate
from megakernels_amd.mixtral.mk import interpret_with_mk
from megakernels_amd.mixtral.scheduler import make_globals, prefill_oproj_barrier
from megakernels_amd.mixtral.synthetic import SMALL, make_synthetic_mixtral
from megakernels_amd.scheduler import tensorize_instructions

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def globs():
    model = make_synthetic_mixtral(SMALL, device="cuda", seed=1)
    return make_globals(model, sm_count=4)


def _launch(g, queues, **kw):
    tensorize_instructions(g, queues)
    g.barriers.zero_()
    prefill_oproj_barrier(g)
    interpret_with_mk(g, mk_mixtral.mk_mixtral, **kw)


def test_missing_arrival_times_out(globs):
    """Opcode 6 with no opcode 5 in any queue: its wait can never complete."""
    queues = [[ExpertDownProjFused(0, 0, 4, 0)], [], [], []]
    with pytest.raises(mk_mixtral.MKDeviceError) as ei:
        _launch(globs, queues, spin_timeout_us=2000, debug_sync=True)
    err = ei.value
    assert err.code == 16 and err.worker == 0 and err.opcode == 6 and err.layer == 0
    assert err.expected == SMALL.intermediate_size // globs.expert_proj_block_size and err.seen == 0
    assert mk_mixtral.read_status("cuda")[0] == 0  # cleared after raising


def test_unsupported_opcode_reported(globs):
    queues = [[Mixtral_QKV(0, 0, 1)], [], [], []]
    with pytest.raises(mk_mixtral.MKDeviceError) as ei:
        _launch(globs, queues, debug_sync=True)
    assert ei.value.code == 18 and ei.value.opcode == 1


def test_bad_operand_reported(globs):
    blocks = SMALL.intermediate_size // globs.expert_proj_block_size
    queues = [[RmsRouterUpgate(0, blocks - 1, 2)], [], [], []]
    with pytest.raises(mk_mixtral.MKDeviceError) as ei:
        _launch(globs, queues, debug_sync=True)
    assert ei.value.code == 19 and ei.value.opcode == 5


def test_failure_stops_waiting_workers(globs):
    """A failure on one worker releases the others blocked on barriers."""
    queues = [[Mixtral_QKV(0, 0, 1)], [ExpertDownProjFused(0, 0, 4, 0)], [], []]
    with pytest.raises(mk_mixtral.MKDeviceError) as ei:
        _launch(globs, queues, spin_timeout_us=10_000_000, debug_sync=True)
    assert ei.value.code == 18


def test_host_validation_rejects_cpu_tensors(globs):
    cpu = make_globals(make_synthetic_mixtral(SMALL, device="cpu", seed=1), sm_count=4)
    tensorize_instructions(cpu, [[], [], [], []])
    with pytest.raises(ValueError):
        interpret_with_mk(cpu, mk_mixtral.mk_mixtral)


def test_recovers_after_error(globs):
    """After a reported failure the next valid launch runs normally."""
    queues = [[Mixtral_QKV(0, 0, 1)], [], [], []]
    with pytest.raises(mk_mixtral.MKDeviceError):
        _launch(globs, queues, debug_sync=True)
    blocks = SMALL.intermediate_size // globs.expert_proj_block_size
    queues = [[RmsRouterUpgate(0, 0, blocks)], [], [], []]
    _launch(globs, queues, debug_sync=True)
    assert int(globs.barriers[0, 4, 0]) == blocks
    torch.cuda.synchronize()
