"""DAG scheduling and per-worker queue tensorisation.

Counterpart of ``megakernels/scheduler.py:13-309``.  A worker is one
workgroup of the persistent kernel (one per compute unit on MI355X); each
worker runs its queue in order and waits on barrier counters in HBM for
cross-worker dependencies.

Assignment strategies keep the reference's semantics:

* ``rr``   instruction ``i`` of the linear (topological) list goes to worker
           ``i % W`` (``megakernels/scheduler.py:155-162``);
* ``zz``   boustrophedon over ``2W`` (``:165-176``);
* ``wave`` consecutive same-opcode runs, each spread by descending cost onto
           the least-loaded worker (``:179-218``);
* ``dag``  list scheduling: ready nodes by descending cost onto the worker
           that frees up first (``:95-152``);
* ``pool`` memory/compute pools by ``tags()['pool']`` (``:221-243``).

``tensorize_instructions`` pads every queue with ``NoOp`` to the longest
length and emits ``instructions[W, Q, 32]`` and ``timings[W, Q, 128]`` int32
(``:275-309``).
"""

from __future__ import annotations

import heapq
from dataclasses import dataclass, field, replace

import torch

from .instructions import BaseGlobals, Instruction, NoOp

INTS_PER_INSTRUCTION = 32
TIMING_SLOTS = 128


@dataclass(eq=False)
class DAG_Node:
    instruction: Instruction
    dependencies: list["DAG_Node"]

    children: list["DAG_Node"] = field(default_factory=list)
    start_time: float = float("inf")
    end_time: float = float("inf")
    priority: float = 0.0

    def earliest_ready_time(self, globs=None) -> float:
        return max((d.end_time for d in self.dependencies), default=0.0)


@dataclass
class Schedule:
    globs: BaseGlobals
    dag_nodes: list[DAG_Node]
    end_node: DAG_Node

    def get_linear_instructions(self) -> list[Instruction]:
        # dag_nodes are built in topological order
        return [n.instruction for n in self.dag_nodes]

    def smart_assign_to_sms(self):
        return assign_dag_to_sms(self)

    def round_robin_assign_to_sms(self):
        return round_robin_assign_to_sms(
            self.get_linear_instructions(), self.globs.sm_count()
        )


class ScheduleBuilder:
    @classmethod
    def make_globals(cls, model, seq_len: int = 0):
        raise NotImplementedError

    @classmethod
    def make_dag(cls, globs, stop_after_op: str | None = None, layer_limit: int | None = None):
        raise NotImplementedError

    @classmethod
    def build(cls, model, stop_after_op: str | None = None, layer_limit: int | None = None, seq_len: int = 0):
        globs = cls.make_globals(model, seq_len=seq_len)
        nodes, end = cls.make_dag(globs, stop_after_op, layer_limit)
        return Schedule(globs, nodes, end)

    @classmethod
    def with_new_globals(cls, schedule: Schedule, model, seq_len: int = 0):
        return replace(schedule, globs=cls.make_globals(model, seq_len=seq_len))


def round_robin_assign_to_sms(instructions: list[Instruction], sm_count: int):
    queues: list[list[Instruction]] = [[] for _ in range(sm_count)]
    for i, ins in enumerate(instructions):
        queues[i % sm_count].append(ins)
    return queues


def zig_zag_assign_to_sms(instructions: list[Instruction], sm_count: int):
    queues: list[list[Instruction]] = [[] for _ in range(sm_count)]
    period = 2 * sm_count
    for i, ins in enumerate(instructions):
        pos = i % period
        w = pos if pos < sm_count else period - 1 - pos
        queues[w].append(ins)
    return queues


def collect_into_waves(instructions: list[Instruction]) -> list[list[Instruction]]:
    """Split the linear list into maximal runs of equal opcode."""
    waves: list[list[Instruction]] = []
    for ins in instructions:
        if waves and waves[-1][-1].opcode() == ins.opcode():
            waves[-1].append(ins)
        else:
            waves.append([ins])
    return waves


def wave_assign_to_sms(schedule: Schedule):
    globs = schedule.globs
    w = globs.sm_count()
    queues: list[list[Instruction]] = [[] for _ in range(w)]
    load = [(0.0, i) for i in range(w)]
    heapq.heapify(load)
    for wave in collect_into_waves(schedule.get_linear_instructions()):
        for ins in sorted(wave, key=lambda x: x.cost(globs), reverse=True):
            t, wid = heapq.heappop(load)
            queues[wid].append(ins)
            heapq.heappush(load, (t + ins.cost(globs), wid))
    return queues


def assign_dag_to_sms(schedule: Schedule):
    """Greedy list scheduling over the DAG (largest ready cost first, onto the
    worker whose queue frees up earliest)."""
    globs = schedule.globs
    nodes = schedule.dag_nodes
    index = {id(n): i for i, n in enumerate(nodes)}
    children: list[list[int]] = [[] for _ in nodes]
    pending = [0] * len(nodes)
    for i, n in enumerate(nodes):
        deps = {id(d) for d in n.dependencies if id(d) in index}
        pending[i] = len(deps)
        for d in deps:
            children[index[d]].append(i)

    w = globs.sm_count()
    queues: list[list[Instruction]] = [[] for _ in range(w)]
    free_at = [(0.0, i) for i in range(w)]
    heapq.heapify(free_at)
    ready = [(-nodes[i].instruction.cost(globs), i) for i in range(len(nodes)) if pending[i] == 0]
    heapq.heapify(ready)
    while ready:
        _, i = heapq.heappop(ready)
        t, wid = heapq.heappop(free_at)
        node = nodes[i]
        node.start_time = t
        node.end_time = t + node.instruction.cost(globs)
        queues[wid].append(node.instruction)
        heapq.heappush(free_at, (node.end_time, wid))
        for c in children[i]:
            pending[c] -= 1
            if pending[c] == 0:
                heapq.heappush(ready, (-nodes[c].instruction.cost(globs), c))
    return queues


def pool_assign_to_sms(instructions: list[Instruction], sm_count: int, memory_fraction: float):
    mem, comp = [], []
    for ins in instructions:
        pool = ins.tags().get("pool")
        if pool == "memory":
            mem.append(ins)
        elif pool == "compute":
            comp.append(ins)
        else:
            raise ValueError(f"Unknown pool: {pool}")
    mem_workers = round(sm_count * memory_fraction)
    return round_robin_assign_to_sms(mem, mem_workers) + round_robin_assign_to_sms(
        comp, sm_count - mem_workers
    )


def assign_to_sms(
    mode: str,
    schedule: Schedule | None = None,
    instructions: list[Instruction] | None = None,
    sm_count: int | None = None,
    memory_fraction: float | None = None,
):
    if schedule is not None:
        instructions = schedule.get_linear_instructions()
        sm_count = schedule.globs.sm_count()
    if mode == "rr":
        return round_robin_assign_to_sms(instructions, sm_count)
    if mode == "zz":
        return zig_zag_assign_to_sms(instructions, sm_count)
    if mode == "wave":
        return wave_assign_to_sms(schedule)
    if mode == "dag":
        return assign_dag_to_sms(schedule)
    if mode == "pool":
        if memory_fraction is None:
            raise ValueError("pool assignment needs memory_fraction")
        return pool_assign_to_sms(instructions, sm_count, memory_fraction)
    raise ValueError(f"Unknown mode: {mode}")


def _row_start(ins: Instruction) -> int:
    for name in ("start_block_idx", "start_output_block_idx"):
        if hasattr(ins, name):
            return getattr(ins, name)
    raise ValueError(f"{type(ins).__name__} has no start block")


def group_rows_by_xcd(queues: list[list[Instruction]], opcodes, xcds: int = 8) -> list[list[Instruction]]:
    """MI355X placement (no reference counterpart): the workgroup of worker
    w runs on XCD ``w % xcds``.  For each opcode in ``opcodes`` and layer,
    the instructions keep their queue positions but trade row ranges, so
    that the workers of one XCD take one contiguous span of rows: the
    instructions in row order go to the positions ordered by (XCD, worker,
    queue slot).  Every position keeps an instruction of the same opcode and
    layer, so the queues' structure and the barrier counts are unchanged;
    only which worker streams which rows changes (instructions of one
    opcode and layer need not have equal block counts)."""
    opcodes = tuple(opcodes)
    slots: dict[tuple[int, int], list[tuple[int, int]]] = {}
    for w, q in enumerate(queues):
        for i, ins in enumerate(q):
            if ins.opcode() in opcodes:
                slots.setdefault((ins.opcode(), ins.layer_idx), []).append((w, i))
    out = [list(q) for q in queues]
    for pos in slots.values():
        items = sorted((queues[w][i] for w, i in pos), key=_row_start)
        order = sorted(pos, key=lambda wi: (wi[0] % xcds, wi[0] // xcds, wi[1]))
        for ins, (w, i) in zip(items, order):
            out[w][i] = ins
    return out


def serialize_and_pad(instruction: Instruction) -> list[int]:
    words = instruction.serialize()
    if len(words) > INTS_PER_INSTRUCTION:
        raise ValueError(
            f"{type(instruction).__name__} serialises to {len(words)} words "
            f"(> {INTS_PER_INSTRUCTION})"
        )
    return words + [0] * (INTS_PER_INSTRUCTION - len(words))


def tensorize_instructions(globs: BaseGlobals, instruction_queues: list[list[Instruction]]):
    """Pad queues with NoOp, serialise, and attach ``instructions [W,Q,32]``
    and ``timings [W,Q,128]`` (int32, on ``globs.device``) to ``globs``."""
    w = globs.sm_count()
    if len(instruction_queues) != w:
        raise ValueError(f"{len(instruction_queues)} queues for {w} workers")
    depth = max((len(q) for q in instruction_queues), default=0)
    depth = max(depth, 1)
    for q in instruction_queues:
        q.extend(NoOp() for _ in range(depth - len(q)))
    flat = [serialize_and_pad(ins) for q in instruction_queues for ins in q]
    globs.instructions = torch.tensor(flat, dtype=torch.int32).view(w, depth, INTS_PER_INSTRUCTION).to(globs.device)
    globs.timings = torch.zeros([w, depth, TIMING_SLOTS], dtype=torch.int32, device=globs.device)
    return globs.instructions
