"""Speed-weighted row partitions for the MoE opcodes.

The reference splits the FFN rows of opcode 5 and the hidden rows of opcode 6
evenly over the workers (``megakernels/mixtral/scheduler.py:176-225``).  On
MI355X the workers do not stream equally fast: workgroup ``w`` runs on XCD
``w % 8``, and the XCDs stream opcode-5 weights at different speeds (one
XCD ends opcode 5 up to ~6 us after another in the kernel's timing record;
the pattern follows the workgroup, not the addresses it reads, and varies
between boxes).  Opcode 6, which every worker starts together after the
barrier, ends evenly across XCDs, so ``opcodes=(5,)`` re-splits opcode 5
only.  Every instruction of an
opcode-5 or opcode-6 set must finish before its consumer starts, so the
slowest worker sets the pace.

``rebalance_queues`` keeps the assignment of instructions to workers and only
moves the block boundaries: the blocks of each (layer, opcode) set are
re-split in their original order in proportion to the speed of the worker
each instruction landed on.  The union of the blocks, the instruction count,
the queue layout and the barrier totals are unchanged, and the results do not
depend on the partition (each output row is computed by exactly one
instruction either way).

``measure_worker_rates`` derives the per-worker speeds from the timing
record of a few launches (``record_timings=True``): rows of opcode 5 streamed
per microsecond between the first weight load and the instruction's
completion.
"""

from __future__ import annotations

import numpy as np
import torch

from .instructions import ExpertDownProjFused, MixtralGlobals, RmsRouterUpgate

# timing-record slots written by the kernel (include/mk_mixtral.h)
_T_FIRST_LOAD = 48
_T_DONE_STORE = 47
_TICKS_PER_US = 100.0


def weighted_spans(num_blocks: int, weights) -> list[tuple[int, int]]:
    """Contiguous (start, end) block spans, one per weight, covering
    ``[0, num_blocks)``, with span sizes proportional to the weights
    (cumulative rounding, so the sizes differ from the ideal by < 1 block)."""
    w = np.asarray(weights, dtype=np.float64)
    if w.ndim != 1 or w.size == 0 or not np.all(np.isfinite(w)) or np.any(w <= 0):
        raise ValueError("weights must be a non-empty vector of positive numbers")
    cum = np.cumsum(w) / w.sum() * num_blocks
    ends = [int(round(c)) for c in cum]
    ends[-1] = num_blocks
    spans, prev = [], 0
    for e in ends:
        e = max(prev, min(e, num_blocks))
        spans.append((prev, e))
        prev = e
    return spans


def rebalance_queues(queues: list[list], globs: MixtralGlobals, worker_weights, opcodes=(5, 6)) -> list[list]:
    """Return new queues whose opcode-5 and opcode-6 instructions (those
    whose opcode is in ``opcodes``) cover the same blocks in the same order,
    re-split by ``worker_weights[worker]``.  The weights measured on opcode 5
    need not hold for opcode 6: all workers start it together after the
    barrier, and its per-XCD end times are even."""
    weights = np.asarray(worker_weights, dtype=np.float64)
    if weights.shape != (len(queues),):
        raise ValueError(f"need one weight per worker ({len(queues)}), got shape {weights.shape}")
    out = [list(q) for q in queues]
    sets: dict[tuple[int, int], list[tuple[int, int, object]]] = {}
    for w, q in enumerate(out):
        for s, ins in enumerate(q):
            if isinstance(ins, (RmsRouterUpgate, ExpertDownProjFused)) and ins.opcode() in opcodes:
                sets.setdefault((ins.opcode(), ins.layer_idx), []).append((w, s, ins))
    for (op, layer), members in sets.items():
        if op == RmsRouterUpgate.opcode():
            members.sort(key=lambda m: m[2].start_block_idx)
            lo = members[0][2].start_block_idx
            hi = max(m[2].start_block_idx + m[2].num_blocks for m in members)
            covered = sum(m[2].num_blocks for m in members)
        else:
            members.sort(key=lambda m: m[2].start_block_idx)
            lo = members[0][2].start_block_idx
            hi = max(m[2].end_block_idx for m in members)
            covered = sum(m[2].end_block_idx - m[2].start_block_idx for m in members)
        if covered != hi - lo:
            raise ValueError(f"opcode {op} layer {layer}: instructions do not tile [{lo}, {hi}) once")
        spans = weighted_spans(hi - lo, [weights[w] for w, _, _ in members])
        for (w, s, ins), (a, b) in zip(members, spans):
            if op == RmsRouterUpgate.opcode():
                out[w][s] = RmsRouterUpgate(layer_idx=layer, start_block_idx=lo + a, num_blocks=b - a)
            else:
                out[w][s] = ExpertDownProjFused(layer_idx=layer, start_block_idx=lo + a, end_block_idx=lo + b,
                                                reduction_block_idx=ins.reduction_block_idx)
    return out


def worker_rates_from_timings(timings: torch.Tensor, instructions: torch.Tensor, expert_proj_block_size: int):
    """Opcode-5 rows per microsecond for each worker from one launch's timing
    record (``timings[W, Q, 128]``, ``instructions[W, Q, 32]``); NaN where a
    worker ran no opcode-5 rows."""
    t = timings.detach().cpu().to(torch.int64) & 0xFFFFFFFF
    ins = instructions.detach().cpu()
    W, Q = ins.shape[0], ins.shape[1]
    rows = np.zeros(W)
    us = np.zeros(W)
    for w in range(W):
        for q in range(Q):
            if int(ins[w, q, 0]) == RmsRouterUpgate.opcode() and int(ins[w, q, 3]) > 0:
                rows[w] += int(ins[w, q, 3]) * expert_proj_block_size
                dt = int(t[w, q, _T_DONE_STORE] - t[w, q, _T_FIRST_LOAD]) & 0xFFFFFFFF
                us[w] += dt / _TICKS_PER_US
    with np.errstate(invalid="ignore", divide="ignore"):
        return np.where((rows > 0) & (us > 0), rows / us, np.nan)


def weights_from_rates(rates, xcds: int = 8, per_worker_blend: float = 0.5) -> np.ndarray:
    """Normalised worker weights from measured rates: a blend of each
    worker's own rate and the mean rate of its XCD (workgroup ``w`` on XCD
    ``w % xcds``), which damps single-launch noise.  Workers without a
    measurement get their XCD's mean."""
    r = np.asarray(rates, dtype=np.float64)
    W = r.size
    xcd = np.arange(W) % xcds
    fallback = np.nanmean(r) if np.any(np.isfinite(r)) else 1.0
    xmean = np.array([np.nanmean(r[xcd == x]) if np.any(np.isfinite(r[xcd == x])) else fallback
                      for x in range(xcds)])
    own = np.where(np.isfinite(r), r, xmean[xcd])
    w = per_worker_blend * own + (1.0 - per_worker_blend) * xmean[xcd]
    return w / w.mean()
