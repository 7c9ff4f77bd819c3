"""CPU emulation of the persistent kernel's dependency protocol.

The HIP kernel runs queue ``w`` of ``instructions[W, Q, 32]`` on worker ``w``
in order.  An instruction first waits until its producer counter reaches the
expected arrival count, then runs, then adds its own arrivals.  A wait that
never completes ends in ``MK_ERR_TIMEOUT`` on the GPU; an opcode the kernel
does not implement ends in ``MK_ERR_UNSUPPORTED_OPCODE``/``MK_ERR_BAD_OPCODE``.

:func:`simulate` replays exactly that control flow on the host (workers
interleaved until none can make progress) and returns the final barrier
tensor, or raises :class:`ProtocolError` carrying the same fields the kernel
writes into its status words.  It needs no GPU, so schedules can be checked
before launch and failure paths can be tested on the CPU.

Counters and arrival counts follow ``megakernels/mixtral/python_vm.py:38-54``
and the arrivals of ``:277, :312-314, :371``.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

MK_ERR_TIMEOUT = 16
MK_ERR_BAD_OPCODE = 17
MK_ERR_UNSUPPORTED_OPCODE = 18
MK_ERR_BAD_INSTRUCTION = 19


@dataclass
class ProtocolDims:
    num_layers: int
    hidden_size: int
    intermediate_size: int
    num_experts_per_tok: int
    expert_proj_block_size: int
    down_proj_block_size: int
    o_proj_block_size: int

    @classmethod
    def from_globals(cls, globs) -> "ProtocolDims":
        return cls(globs.num_hidden_layers, globs.hidden_size, globs.intermediate_size,
                   globs.num_experts_per_tok, globs.expert_proj_block_size,
                   globs.down_proj_block_size, globs.o_proj_block_size)


class ProtocolError(RuntimeError):
    def __init__(self, code, worker, slot, opcode, layer, expected, seen):
        self.code, self.worker, self.slot = code, worker, slot
        self.opcode, self.layer, self.expected, self.seen = opcode, layer, expected, seen
        super().__init__(
            f"code {code} at worker {worker} slot {slot} opcode {opcode} layer {layer} "
            f"(expected {expected}, seen {seen})"
        )


def _wait_and_arrive(words, d: ProtocolDims):
    """(wait (layer, op_row, expected) or None, arrive (layer, op_row, n), error) for one instruction."""
    op = int(words[0])
    if op == 0:
        return None, None, None
    if op in (1, 2, 3, 4, 7):
        return None, None, (MK_ERR_UNSUPPORTED_OPCODE, int(words[1]), 0, op)
    if op == 5:
        layer, start, nb = (int(x) for x in words[1:4])
        if not (0 <= layer < d.num_layers and start >= 0 and nb >= 0
                and (start + nb) * d.expert_proj_block_size <= d.intermediate_size):
            return None, None, (MK_ERR_BAD_INSTRUCTION, layer, start, nb)
        return (layer, 3, d.hidden_size // d.o_proj_block_size), (layer, 4, nb), None
    if op == 6:
        layer, start, end, red = (int(x) for x in words[1:5])
        if not (0 <= layer < d.num_layers and 0 <= start <= end
                and end * d.down_proj_block_size <= d.hidden_size and red == 0):
            return None, None, (MK_ERR_BAD_INSTRUCTION, layer, start, end)
        return ((layer, 4, d.intermediate_size // d.expert_proj_block_size),
                (layer, 5, d.num_experts_per_tok * (end - start)), None)
    if op == 8:
        layer = int(words[1])
        if not 0 <= layer < d.num_layers:
            return None, None, (MK_ERR_BAD_INSTRUCTION, layer, 0, 0)
        wait = None
        if layer > 0:
            wait = (layer - 1, 5, d.num_experts_per_tok * (d.hidden_size // d.down_proj_block_size))
        return wait, (layer, 7, 1), None
    return None, None, (MK_ERR_BAD_OPCODE, 0, 0, op)


def _as_numpy(a) -> np.ndarray:
    if hasattr(a, "detach"):  # torch tensor, possibly on a GPU
        return a.detach().cpu().numpy()
    return np.asarray(a)


def simulate(instructions, barriers, dims: ProtocolDims) -> np.ndarray:
    """Replay the queues; return the final barrier tensor (a copy).

    ``instructions`` is ``[W, Q, 32]`` and ``barriers`` ``[L, ops, width]``
    (numpy arrays or CPU tensors).  Raises :class:`ProtocolError` for the
    first failure the kernel would report: an invalid instruction as soon as
    its worker reaches it, or -- when no worker can progress -- a time-out of
    the lowest-numbered blocked worker.
    """
    ins = _as_numpy(instructions).astype(np.int64)
    bar = _as_numpy(barriers).astype(np.int64, copy=True)
    W, Q, _ = ins.shape
    pos = [0] * W
    decoded = [[_wait_and_arrive(ins[w, q], dims) for q in range(Q)] for w in range(W)]
    while True:
        progressed = False
        for w in range(W):
            while pos[w] < Q:
                wait, arrive, err = decoded[w][pos[w]]
                if err is not None:
                    code, layer, a, b = err
                    op = int(ins[w, pos[w], 0])
                    raise ProtocolError(code, w, pos[w], op, layer, a, b)
                if wait is not None and bar[wait[0], wait[1], 0] < wait[2]:
                    break
                if arrive is not None:
                    bar[arrive[0], arrive[1], 0] += arrive[2]
                pos[w] += 1
                progressed = True
        if all(p == Q for p in pos):
            return bar
        if not progressed:
            w = min(i for i in range(W) if pos[i] < Q)
            wait, _, _ = decoded[w][pos[w]]
            raise ProtocolError(MK_ERR_TIMEOUT, w, pos[w], int(ins[w, pos[w], 0]), wait[0], wait[2],
                                int(bar[wait[0], wait[1], 0]))

