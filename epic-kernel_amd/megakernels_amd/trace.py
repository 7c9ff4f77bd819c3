"""Analysis of the persistent kernel's timing record.

With ``record_timings=True`` the kernel writes, per instruction slot
``timings[w, q, :]``, 32-bit ``s_memrealtime`` stamps (100 MHz, one clock
shared by all compute units) at the slot indices of the reference's timing
convention (``include/util.cuh:220-252``):

* 0 / 4    instruction start / end
* 44 / 45  barrier wait entered / satisfied
* 46       own items done (work sharing; opcode 2: wave 0's positions)
* 47       instruction's stores complete and arrival made
* 48       first weight load issued
* 49       first staged data in place (opcode 2: its K/V ring has landed;
           opcode 5: speculative expert loads issued)
* 50       opcode 5 of a whole-model launch: predicted and selected experts
           (bytes p0, p1, s0, s1; 0xff = no prediction), not a time

This module turns that record into what the reference's plotting scripts
derive from theirs, as numbers rather than figures:

* :func:`barrier_waits` -- per-opcode and per-layer barrier wait time, the
  quantity of ``megakernels/scripts/plot_barrier_waits.py:131-212``;
* :func:`hbm_utilization` -- aggregate weight-streaming bandwidth over time:
  each instruction's algorithmic bytes spread evenly over its streaming
  window (first load to completion), summed over workers and binned, the
  method of ``megakernels/scripts/plot_hbm_utilization.py:87-212``;
* :func:`phase_summary` -- percentiles of the event times across workers.

Records are saved with :func:`save_record` as ``.npz`` (no pickling).
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import numpy as np

TICKS_PER_US = 100.0
T_START, T_END = 0, 4
T_AT_WAIT, T_DONE_WAIT = 44, 45
T_OWN_DONE, T_DONE_STORE, T_FIRST_LOAD, T_FIRST_USE = 46, 47, 48, 49

OPCODE_NAMES = {
    1: "QKV",
    2: "PartialAttn",
    3: "AttnReduction",
    4: "OProj",
    5: "RmsRouterUpgate",
    6: "ExpertDownProjFused",
    7: "RMS_LM_Head",
    8: "SpeculativeExpertPredict",
}

#: opcode names of the dense (Llama) VM, megakernels/demos/latency/instructions.py
DENSE_OPCODE_NAMES = {
    1: "QKV",
    2: "PartialAttn",
    3: "AttnReduction",
    4: "OProj",
    5: "UpGateSiLU",
    6: "DownProjResidual",
    7: "RMS_LM_Head",
}


@dataclass
class TimingRecord:
    """``timings[W, Q, 128]`` and ``instructions[W, Q, 32]`` (int32) of one
    launch, plus the shape constants needed for the byte model."""

    timings: np.ndarray
    instructions: np.ndarray
    hidden_size: int
    intermediate_size: int
    num_experts: int
    expert_proj_block_size: int
    down_proj_block_size: int
    k: int = 2
    qkv_block_size: int = 0
    o_proj_block_size: int = 0
    lm_head_block_size: int = 0
    attn_width: int = 0  # Hq * head_dim, the O-projection's reduction length
    head_dim: int = 0
    num_kv_heads: int = 0
    attn_kv_block_size: int = 0
    pos_id: int = 0
    red_cols: int = 0  # dense VM: down-projection column chunk; 0 for Mixtral

    @property
    def dense(self) -> bool:
        return self.red_cols > 0

    @property
    def opcode_names(self) -> dict:
        return DENSE_OPCODE_NAMES if self.dense else OPCODE_NAMES

    @classmethod
    def from_globals(cls, globs) -> "TimingRecord":
        dense = hasattr(globs, "up_gate_proj_block_size")
        return cls(
            timings=globs.timings.detach().cpu().numpy().copy(),
            instructions=globs.instructions.detach().cpu().numpy().copy(),
            hidden_size=globs.hidden_size,
            intermediate_size=globs.intermediate_size,
            num_experts=1 if dense else globs.num_experts,
            expert_proj_block_size=globs.up_gate_proj_block_size if dense else globs.expert_proj_block_size,
            down_proj_block_size=globs.down_proj_block_size,
            k=1 if dense else globs.num_experts_per_tok,
            red_cols=globs.matvec_reduction_size if dense else 0,
            qkv_block_size=globs.qkv_block_size,
            o_proj_block_size=globs.o_proj_block_size,
            lm_head_block_size=globs.lm_head_block_size,
            attn_width=globs.num_attention_heads * globs.head_dim,
            head_dim=globs.head_dim,
            num_kv_heads=globs.num_kv_heads,
            attn_kv_block_size=globs.attn_kv_block_size,
            pos_id=int(globs.pos_id),
        )

    def micros(self) -> np.ndarray:
        """Stamps as float microseconds since the earliest instruction start,
        NaN where a stamp was not written.  The 32-bit counter may wrap once
        within a launch; stamps are unwrapped relative to the earliest start."""
        t = self.timings.astype(np.int64) & 0xFFFFFFFF
        ops = self.instructions[:, :, 0]
        busy = ops != 0
        starts = np.unique(t[:, :, T_START][busy & (t[:, :, T_START] != 0)])
        if starts.size == 0:
            return np.full(t.shape, np.nan)
        # the earliest start is the one from which every other start is
        # reached by the shortest forward (modular) distance
        spread = ((starts[None, :] - starts[:, None]) & 0xFFFFFFFF).max(axis=1)
        t0 = int(starts[int(np.argmin(spread))])
        rel = (t - t0) & 0xFFFFFFFF  # modular difference handles one wrap
        out = rel.astype(np.float64) / TICKS_PER_US
        out[t == 0] = np.nan
        out[~busy] = np.nan
        return out

    def streamed_bytes(self, w: int, q: int) -> int:
        """Algorithmic HBM bytes of the instruction at (w, q): the weight rows
        it streams (bf16)."""
        ins = self.instructions[w, q]
        op = int(ins[0])
        H, F, E = self.hidden_size, self.intermediate_size, self.num_experts
        if self.dense and op == 5:
            return int(ins[2]) * self.expert_proj_block_size * H * 2 * 2  # gate + up rows of the listed blocks
        if self.dense and op == 6:
            return (int(ins[3]) - int(ins[2])) * self.down_proj_block_size * self.red_cols * 2
        if self.dense and op == 7:
            return (int(ins[2]) - int(ins[1])) * self.lm_head_block_size * H * 2
        if op == 5:
            rows = int(ins[3]) * self.expert_proj_block_size
            return self.k * 2 * rows * H * 2  # gate + up rows of each selected expert
        if op == 6:
            rows = (int(ins[3]) - int(ins[2])) * self.down_proj_block_size
            return self.k * rows * F * 2
        if op == 8:
            return E * H * 2 + H * 2
        if op == 1 and self.qkv_block_size:
            return (int(ins[3]) - int(ins[2])) * self.qkv_block_size * H * 2
        if op == 2 and self.head_dim and self.attn_kv_block_size:
            # K and V rows of the partition's positions (python_vm.py:125-159
            # split: blocks of attn_kv_block_size over num_partials)
            nparts, pidx = int(ins[3]), int(ins[4])
            seq = self.pos_id + 1
            total = -(-seq // self.attn_kv_block_size)
            per = -(-total // nparts)
            t0 = min(pidx * per, total) * self.attn_kv_block_size
            t1 = min(min(pidx * per + per, total) * self.attn_kv_block_size, seq)
            return max(t1 - t0, 0) * 2 * self.head_dim * 2
        if op == 4 and self.o_proj_block_size:
            return (int(ins[3]) - int(ins[2])) * self.o_proj_block_size * self.attn_width * 2
        if op == 7 and self.lm_head_block_size:
            return (int(ins[2]) - int(ins[1])) * self.lm_head_block_size * 2048 * 2
        return 0


def save_record(path, rec: TimingRecord) -> None:
    np.savez_compressed(
        path, timings=rec.timings, instructions=rec.instructions,
        shape=np.array([rec.hidden_size, rec.intermediate_size, rec.num_experts,
                        rec.expert_proj_block_size, rec.down_proj_block_size, rec.k,
                        rec.qkv_block_size, rec.o_proj_block_size, rec.lm_head_block_size, rec.attn_width,
                        rec.head_dim, rec.num_kv_heads, rec.attn_kv_block_size, rec.pos_id, rec.red_cols]))


def load_record(path) -> TimingRecord:
    d = np.load(Path(path), allow_pickle=False)
    shape = [int(x) for x in d["shape"]] + [0] * 8
    return TimingRecord(d["timings"], d["instructions"], *shape[:15])


def barrier_waits(rec: TimingRecord) -> dict:
    """Per opcode: instruction count, total and mean wait (us), total
    instruction time (us), wait share; per layer: total wait (us) by
    opcode."""
    t = rec.micros()
    ops = rec.instructions[:, :, 0]
    layers = rec.instructions[:, :, 1]
    by_op: dict[int, dict] = {}
    by_layer: dict[int, dict] = {}
    W, Q = ops.shape
    for w in range(W):
        for q in range(Q):
            op = int(ops[w, q])
            if op == 0 or np.isnan(t[w, q, T_START]) or np.isnan(t[w, q, T_END]):
                continue
            wait = t[w, q, T_DONE_WAIT] - t[w, q, T_AT_WAIT]
            wait = 0.0 if np.isnan(wait) else max(0.0, float(wait))
            dur = max(0.0, float(t[w, q, T_END] - t[w, q, T_START]))
            s = by_op.setdefault(op, {"name": rec.opcode_names.get(op, str(op)), "count": 0, "wait_us": 0.0,
                                      "instr_us": 0.0})
            s["count"] += 1
            s["wait_us"] += wait
            s["instr_us"] += dur
            layer = int(layers[w, q]) if op != 7 else -1
            by_layer.setdefault(layer, {}).setdefault(op, 0.0)
            by_layer[layer][op] += wait
    for s in by_op.values():
        s["mean_wait_us"] = s["wait_us"] / s["count"]
        s["wait_share"] = s["wait_us"] / s["instr_us"] if s["instr_us"] > 0 else 0.0
    return {"by_opcode": by_op, "by_layer": by_layer}


def hbm_utilization(rec: TimingRecord, bin_us: float = 1.0, peak_gbs: float = 8000.0):
    """(bin start times [us], aggregate GB/s per bin, fraction of peak per
    bin, total bytes).  Each instruction's bytes are spread uniformly over
    [first load, completion]."""
    t = rec.micros()
    W, Q = rec.instructions.shape[:2]
    spans = []
    for w in range(W):
        for q in range(Q):
            nb = rec.streamed_bytes(w, q)
            a, b = t[w, q, T_FIRST_LOAD], t[w, q, T_DONE_STORE]
            if nb <= 0 or np.isnan(a) or np.isnan(b) or b <= a:
                continue
            spans.append((a, b, nb))
    if not spans:
        return np.zeros(0), np.zeros(0), np.zeros(0), 0
    end = max(b for _, b, _ in spans)
    nbins = int(np.ceil(end / bin_us)) + 1
    edges = np.arange(nbins + 1) * bin_us
    acc = np.zeros(nbins)
    for a, b, nb in spans:
        rate = nb / (b - a)  # bytes per us
        lo = np.clip(edges[:-1], a, b)
        hi = np.clip(edges[1:], a, b)
        acc += rate * (hi - lo)
    gbs = acc / bin_us / 1e3  # bytes/us -> GB/s
    total = int(sum(nb for _, _, nb in spans))
    return edges[:-1], gbs, gbs / peak_gbs, total


def phase_summary(rec: TimingRecord, percentiles=(0, 10, 50, 90, 100)) -> dict:
    """Percentiles over workers of each event time (us), keyed by
    (opcode name, event)."""
    t = rec.micros()
    ops = rec.instructions[:, :, 0]
    events = {"start": T_START, "wait_done": T_DONE_WAIT, "first_load": T_FIRST_LOAD, "first_use": T_FIRST_USE,
              "own_done": T_OWN_DONE, "done": T_DONE_STORE, "end": T_END}
    out = {}
    for op in sorted(set(int(x) for x in np.unique(ops)) - {0}):
        mask = ops == op
        for name, slot in events.items():
            v = t[:, :, slot][mask]
            v = v[~np.isnan(v)]
            if v.size:
                out[(rec.opcode_names.get(op, str(op)), name)] = np.percentile(v, percentiles)
    return out


T_PREDICTION = 50


def prediction_agreement(rec: TimingRecord):
    """Opcode 8's prediction against opcode 5's selection, from the first
    opcode-5 instruction of each layer (every workgroup routes identically):
    (layers with a prediction, top-1 agreement, top-2 set agreement), or None
    when no layer had one."""
    ins = rec.instructions
    seen = {}
    W, Q = ins.shape[:2]
    for w in range(W):
        for q in range(Q):
            if int(ins[w, q, 0]) != 5 or rec.dense:
                continue
            layer = int(ins[w, q, 1])
            if layer in seen:
                continue
            v = int(rec.timings[w, q, T_PREDICTION]) & 0xFFFFFFFF
            p0, p1, s0, s1 = v & 0xFF, (v >> 8) & 0xFF, (v >> 16) & 0xFF, (v >> 24) & 0xFF
            if p0 == 0xFF or v == 0:
                continue
            seen[layer] = (p0, p1, s0, s1)
    if not seen:
        return None
    n = len(seen)
    top1 = sum(p0 == s0 for p0, _, s0, _ in seen.values()) / n
    top2 = sum({p0, p1} == {s0, s1} for p0, p1, s0, s1 in seen.values()) / n
    return n, top1, top2


def stage_windows(rec: TimingRecord) -> dict:
    """Per (layer, opcode): (first start, last end, last completion) in us --
    the critical-path view of a whole-model step (the LM head is layer -1)."""
    t = rec.micros()
    ops = rec.instructions[:, :, 0]
    layers = rec.instructions[:, :, 1]
    out: dict = {}
    W, Q = ops.shape
    for w in range(W):
        for q in range(Q):
            op = int(ops[w, q])
            if op == 0 or np.isnan(t[w, q, T_START]):
                continue
            key = (-1 if op == 7 else int(layers[w, q]), op)
            a, b = t[w, q, T_START], t[w, q, T_END]
            done = t[w, q, T_DONE_STORE]
            lo, hi, dn = out.get(key, (np.inf, -np.inf, -np.inf))
            out[key] = (min(lo, a), max(hi, b), max(dn, done if not np.isnan(done) else b))
    return out


def format_report(rec: TimingRecord, peak_gbs: float = 8000.0) -> str:
    """A plain-text report of the three analyses."""
    lines = []
    bw = barrier_waits(rec)
    lines.append("opcode                      count  mean wait us  wait share")
    for op, s in sorted(bw["by_opcode"].items()):
        lines.append(f"{s['name']:26s} {s['count']:6d}  {s['mean_wait_us']:12.2f}  {s['wait_share']:10.3f}")
    starts, gbs, frac, total = hbm_utilization(rec, peak_gbs=peak_gbs)
    if gbs.size:
        busy = gbs > 0
        lines.append(f"streamed {total / 1e6:.1f} MB over {starts[busy][-1] - starts[busy][0] + 1:.0f} us; "
                     f"peak bin {gbs.max():.0f} GB/s ({frac.max():.1%}), mean over busy bins "
                     f"{gbs[busy].mean():.0f} GB/s ({frac[busy].mean():.1%})")
    win = stage_windows(rec)
    layers = sorted({lay for lay, _ in win if lay >= 0})
    if len(layers) > 1:
        show = layers[len(layers) // 2]
        lines.append(f"layer {show} stage windows (us, first start / last end):")
        for (lay, op), (a, b, _) in sorted(win.items()):
            if lay == show:
                lines.append(f"  {rec.opcode_names.get(op, op):26s} {a:9.1f} {b:9.1f}  ({b - a:6.1f})")
        ends = [max(b for (lay, _), (_, b, _) in win.items() if lay == L) for L in layers]
        if len(ends) > 2:
            lines.append(f"mean layer period {np.mean(np.diff(ends)):.1f} us over {len(layers)} layers")
    agree = prediction_agreement(rec)
    if agree is not None:
        n, top1, top2 = agree
        lines.append(f"expert prediction over {n} layers: top-1 agreement {top1:.1%}, top-2 set agreement {top2:.1%}")
    lines.append("event percentiles (us): p0 p10 p50 p90 p100")
    for (name, ev), v in phase_summary(rec).items():
        lines.append(f"  {name:26s} {ev:10s} " + " ".join(f"{x:7.1f}" for x in v))
    return "\n".join(lines)


if __name__ == "__main__":
    import sys

    for path in sys.argv[1:]:
        print(f"== {path}")
        print(format_report(load_record(path)))
