"""Schedule builders and interpreters by VM name.

Counterpart of ``megakernels/dispatch.py:20-40`` for the VMs this build runs
(the throughput VM is outside the hot path): ``latency`` / ``latency_3b``
(dense Llama) and ``mixtral_latency``.  The CPU solver tables live in the
oracle (test infrastructure) and are not mapped here.
"""

from __future__ import annotations

from .latency.mk import Latency3B_MK_Interpreter, LatencyMK_Interpreter
from .latency.scheduler import LatencyScheduleBuilder
from .mixtral.mk import MixtralMK_Interpreter
from .mixtral.scheduler import MixtralLatencyScheduleBuilder

BUILDER_MAP = {
    "latency": LatencyScheduleBuilder,
    "latency_3b": LatencyScheduleBuilder,
    "mixtral_latency": MixtralLatencyScheduleBuilder,
}

MK_INTERPRETER_MAP = {
    "latency": LatencyMK_Interpreter,
    "latency_3b": Latency3B_MK_Interpreter,
    "mixtral_latency": MixtralMK_Interpreter,
}


def make_schedule_builder(mode: str):
    return BUILDER_MAP[mode]


def make_mk_interpreter(mode: str, mk_dir=None):
    return MK_INTERPRETER_MAP[mode](mk_dir)
