#!/usr/bin/env python3
"""Benchmark: batch-1 Mixtral-8x7B decode on one MI355X.

Headline (the default run): Mixtral-8x7B-shaped batch-1
greedy decode -- 32 layers, hidden 4096, 32/8 heads, 8 experts top-2 with
FFN 14336, vocab 32000, random-init bf16 weights (94 GB, resident in HBM),
the KV cache pre-filled to 4096 positions.  One *step* = one decode token =
one launch of the persistent kernel over the whole model, with the argmax
and the next token's embedding inside the launch.  ``value`` is decode
tokens/s; ``roofline`` is the step's algorithmic bytes (weights, the K/V of
every cached position, the LM head) over the kernel time from HIP events on
the launch stream.

Also in the same line:
* ``moe_layer``: one full-size Mixtral MoE layer in isolation (BASELINE
  config 2): 1024 batch-1 tokens per step, each a launch of opcodes 5 and 6,
  its microseconds per launch, HBM roofline fraction of
  2*(E*H + H + k*3*F*H) bytes, the skewed-routing variant (+2.0 router
  bias on experts 0 and 1) and a same-run correctness gate (8 tokens against
  the CPU oracle);
* ``configs``: configs 5 (the same model at 16384 cached positions, with a
  predictor of router + N(0, sigma) weights, the measured prediction
  agreement and the predictor on/off A/B) and 3 (Llama-3.2-3B shape, dense
  VM), timed in the same run, each with its own roofline;
* ``correctness``: the token and last-layer experts of one whole-model
  launch over a two-layer slice of the headline model against the CPU
  oracle's step of the same slice;
* ``cpu_baseline``: the CPU oracle (a restatement of the reference's
  python_vm; bf16 einsum per block as the reference runs it, and the C +
  OpenMP leg beside it) timed on the host over a bounded slice of the same
  decode workload and scaled to tokens/s.

``python bench.py`` (defaults: 128 timed steps after 2 warmup steps);
``--config c2`` / ``c1`` run the MoE layer alone, ``c3`` / ``c5`` the other
decode configs alone, ``--c4-only`` the headline alone.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT / "epic-kernel_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

METRIC = "batch-1 decode tokens/s, Mixtral-8x7B shape; MoE layer µs; % HBM peak"
HBM_PEAK_GBS = 8000.0
# HBM bytes moved per launch (rocprofv3 FETCH_SIZE and WRITE_SIZE per
# dispatch, each scaled by what the same counter reads for a device copy of
# known size: FETCH x 2.0, WRITE x 1.0), measured on the kernel of commit
# 0e3b696: config 2 one MoE layer; configs 3/4/5 one decode step at 2050 /
# 4098 / 16386 cached positions.  The counter runs are summarised under
# profiles/.
MEASURED_TRAFFIC_BYTES = {"c2": 707_841_102, "c3": 6_749_136_490, "c4": 26_290_541_573, "c5": 28_033_287_742}
TRAFFIC_UNIT = ("bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated, kernel of commit 0e3b696; "
                "configs 3-5 at 2050 / 4098 / 16386 cached positions)")


def moe_layer_bytes(cfg) -> int:
    """Algorithmic HBM bytes of one MoE layer: router + ffn RMSNorm weights +
    k experts x {gate, up, down}, bf16."""
    E, H, F, k = cfg.num_local_experts, cfg.hidden_size, cfg.intermediate_size, cfg.num_experts_per_tok
    return 2 * (E * H + H + k * 3 * F * H)


def cpu_model_name() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


class MoEBench:
    """Per-token launches of the MoE-only schedule over resident inputs."""

    def __init__(self, cfg, tokens: int, seed: int = 0, router_bias=None, work_sharing: bool = False,
                 balance: bool = False, calib_tokens: int = 16, moe_overlap: str = "off", upgate_rounds: int = 3,
                 balance_opcodes=(5, 6)):
        import torch

        import mk_mixtral
        from megakernels_amd.mixtral.scheduler import make_globals, make_moe_dag, expected_oproj_arrivals
        from megakernels_amd.mixtral.synthetic import make_residuals, make_synthetic_mixtral
        from megakernels_amd.scheduler import Schedule, assign_to_sms, tensorize_instructions

        self.torch = torch
        self.dev = torch.device("cuda:0")
        self.cfg = cfg
        self.tokens = tokens
        self.model = make_synthetic_mixtral(cfg, self.dev, seed, router_bias=router_bias)
        self.residuals = make_residuals(tokens, cfg.hidden_size, generator=self.model.generator)
        # speed-balanced partitions need row-granular blocks
        self.balance_opcodes = tuple(balance_opcodes)
        bs = {}
        if balance:
            bs["expert_proj_block_size"] = 1
            if 6 in self.balance_opcodes:
                bs["down_proj_block_size"] = 1
        self.globs = g = make_globals(self.model, moe_overlap=moe_overlap in ("on", "op5"),
                                      upgate_rounds=upgate_rounds, **bs)
        nodes, end = make_moe_dag(g)
        self.schedule = Schedule(g, nodes, end)
        self.queues = assign_to_sms("rr", schedule=self.schedule)
        tensorize_instructions(g, self.queues)
        # one barrier tensor and one residual row per token, so a step needs
        # no per-token resets between launches
        bars = torch.zeros([tokens, *g.barriers.shape], dtype=torch.int32, device=self.dev)
        bars[:, 0, 3, 0] = expected_oproj_arrivals(g)
        self.bars_init = bars
        self.bars = bars.clone()
        self.work = self.residuals.clone()

        from megakernels_amd.mixtral.mk import interpret_with_mk

        captured = {}

        def capture(*args, **kw):
            kw.pop("stream", None)
            captured["g"] = mk_mixtral.build_globals_struct(*args, **kw)

        interpret_with_mk(g, capture, work_sharing=work_sharing, downproj_overlap=moe_overlap in ("on", "op6"))
        self.struct = captured["g"]
        self.lib = mk_mixtral.load_library()
        self.mk = mk_mixtral
        self.row_bytes = self.work.stride(0) * 2
        self.bar_bytes = self.bars.stride(0) * 4
        self.weights = None
        if balance:
            self.calibrate(calib_tokens)

    def calibrate(self, n: int):
        """Measure each worker's opcode-5 streaming rate on `n` launches (timing
        record on), then re-split the opcode-5/6 rows by speed."""
        import numpy as np

        from megakernels_amd.mixtral.balance import rebalance_queues, weights_from_rates, worker_rates_from_timings
        from megakernels_amd.scheduler import tensorize_instructions

        torch, g, s = self.torch, self.globs, self.struct
        s.record_timings = 1
        s.timings = g.timings.data_ptr()
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        self.work.copy_(self.residuals)
        self.bars.copy_(self.bars_init)
        rates = []
        for t in range(n + 2):
            self._launch(t % self.tokens, stream)
            torch.cuda.synchronize()
            if t >= 2:  # first launches warm up
                rates.append(worker_rates_from_timings(g.timings, g.instructions, g.expert_proj_block_size))
        self.check_status()
        self.weights = weights_from_rates(np.nanmean(np.stack(rates), axis=0))
        self.queues = rebalance_queues(self.queues, g, self.weights, opcodes=self.balance_opcodes)
        tensorize_instructions(g, self.queues)
        s.instructions = g.instructions.data_ptr()
        s.queue_len = g.instructions.shape[1]
        s.record_timings = 0
        s.timings = g.timings.data_ptr()

    def linear_instructions(self):
        """The launched instructions in topological order (round-robin
        assignment: linear index i sits at queue i % W, position i // W)."""
        W = len(self.queues)
        n = len(self.schedule.get_linear_instructions())
        return [self.queues[i % W][i // W] for i in range(n)]

    def _launch(self, t: int, stream_ptr):
        s = self.struct
        s.hidden_states = self.work.data_ptr() + t * self.row_bytes
        s.barriers = self.bars.data_ptr() + t * self.bar_bytes
        rc = self.lib.mk_mixtral_launch(ctypes.byref(s), stream_ptr)
        if rc:
            raise self.mk.MKError(rc, self.lib.mk_mixtral_error_string(rc).decode())

    def step(self):
        self.work.copy_(self.residuals)
        self.bars.copy_(self.bars_init)
        stream = ctypes.c_void_p(self.torch.cuda.current_stream(self.dev).cuda_stream)
        for t in range(self.tokens):
            self._launch(t, stream)

    def per_launch_us(self, n: int):
        """Event-timed individual launches (median/p10/p90 in microseconds)."""
        torch = self.torch
        self.work.copy_(self.residuals)
        self.bars.copy_(self.bars_init)
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        for t in range(n):
            evs[t][0].record()
            self._launch(t % self.tokens, stream)
            evs[t][1].record()
        torch.cuda.synchronize()
        us = sorted(a.elapsed_time(b) * 1e3 for a, b in evs)
        return {"median": statistics.median(us), "p10": us[int(0.1 * (n - 1))], "p90": us[int(0.9 * (n - 1))],
                "min": us[0]}

    def check_status(self):
        self.mk.raise_if_failed(self.dev)


def run_timed(bench, steps: int, warmup: int):
    torch = bench.torch
    for _ in range(warmup):
        bench.step()
    torch.cuda.synchronize()
    bench.check_status()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        bench.step()
    stop.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    bench.check_status()
    wall = t1 - t0
    launches = steps * bench.tokens
    gpu_s = start.elapsed_time(stop) / 1e3
    return {"wall_s": wall, "gpu_s": gpu_s, "launches": launches, "us_per_launch_events": gpu_s / launches * 1e6}


def record_trace(bench, path: str, launches: int = 8):
    """Launch `launches` tokens with the timing record on (after the timed
    region, so it does not perturb the measurement), save the last record."""
    from megakernels_amd.trace import TimingRecord, format_report, save_record

    torch, g, s = bench.torch, bench.globs, bench.struct
    s.record_timings = 1
    s.timings = g.timings.data_ptr()
    stream = ctypes.c_void_p(torch.cuda.current_stream(bench.dev).cuda_stream)
    bench.work.copy_(bench.residuals)
    bench.bars.copy_(bench.bars_init)
    for t in range(launches):
        g.timings.zero_()
        bench._launch(t % bench.tokens, stream)
    torch.cuda.synchronize()
    bench.check_status()
    s.record_timings = 0
    rec = TimingRecord.from_globals(g)
    save_record(path, rec)
    print(format_report(rec), file=sys.stderr, flush=True)


def decode_bytes_per_token(cfg, seq_len: int) -> int:
    """Algorithmic HBM bytes of one whole-model decode step: every layer's
    attention weights, norms, router and the two selected experts, the K and
    V rows of all cached positions, and the LM head with its norm (bf16)."""
    L, H, F, E, k = (cfg.num_hidden_layers, cfg.hidden_size, cfg.intermediate_size, cfg.num_local_experts,
                     cfg.num_experts_per_tok)
    Hq, Hkv, D, V = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.vocab_size
    attn = (Hq + 2 * Hkv) * D * H + H * Hq * D + H
    moe = E * H + H + k * 3 * F * H
    kv = 2 * seq_len * Hkv * D
    return 2 * (L * (attn + moe + kv) + V * H + H)


def decode_bytes_per_token_llama(cfg, seq_len: int) -> int:
    """Algorithmic HBM bytes of one dense (Llama) decode step: every layer's
    QKV, O, up, gate and down projections with both norms, the K and V rows
    of all cached positions, and the LM head with its norm (bf16)."""
    L, H, F = cfg.num_hidden_layers, cfg.hidden_size, cfg.intermediate_size
    Hq, Hkv, D, V = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.vocab_size
    attn = (Hq + 2 * Hkv) * D * H + H * Hq * D + H
    mlp = 3 * F * H + H
    kv = 2 * seq_len * Hkv * D
    return 2 * (L * (attn + mlp + kv) + V * H + H)


#: BASELINE config 5: predictor weights = router + N(0, sigma), sigma tuned
#: for ~80 % top-2 agreement with the true router: a sweep at 16384 cached
#: positions (``--config c5 --sigma-sweep``, 8 steps x 32 layers each) gave
#: top-2 set agreement 99.2 / 92.2 / 81.6 / 76.2 / 70.7 / 62.1 % at sigma 0 /
#: 0.002 / 0.003 / 0.004 / 0.005 / 0.007; the agreement measured in the run
#: is reported in the bench line
C5_SIGMA = 0.003
PREFILL = {"c3": 2048, "c4": 4096, "c5": 16384}


def build_decode_model(config: str, positions: int, sigma: float | None, prefill: int | None = None):
    """Random-init weights resident in HBM (seed 0) and a KV cache pre-filled
    with N(0, 1) to ``prefill`` positions (default: the config's context),
    with room for ``positions`` positions in all."""
    import torch

    prefill = PREFILL[config] if prefill is None else prefill
    t0 = time.perf_counter()
    if config == "c3":
        from megakernels_amd.latency.synthetic import C3, make_synthetic_llama

        cfg = C3
        print(f"bench: building c3 ({cfg.num_hidden_layers} layers, {prefill} cached positions) on cuda:0",
              file=sys.stderr, flush=True)
        model = make_synthetic_llama(cfg, "cuda", 0, kv_positions=positions, prefill=prefill)
    else:
        from megakernels_amd.mixtral.synthetic import C4, make_synthetic_mixtral

        cfg = C4
        print(f"bench: building the Mixtral model ({cfg.num_hidden_layers} layers, {prefill} cached positions) "
              "on cuda:0", file=sys.stderr, flush=True)
        model = make_synthetic_mixtral(cfg, "cuda", 0, full=True, kv_positions=positions, prefill=prefill,
                                       predictor_sigma=sigma)
    torch.cuda.synchronize()
    print(f"bench: weights ready in {time.perf_counter() - t0:.0f} s, {torch.cuda.memory_allocated() / 1e9:.1f} GB "
          "allocated", file=sys.stderr, flush=True)
    return model


def decode_bench(args, config: str, steps: int, warmup: int, model=None, sigma: float | None = None,
                 prefetch_rounds: int | None = None):
    """Whole-model greedy decode through MK_Generator
    (Llama-3.2-3B shape, 2048 cached positions, dense VM) and configs 4 and 5
    (Mixtral-8x7B shape, 4096 / 16384 cached positions).  Random-init weights
    resident in HBM, a KV cache pre-filled with N(0, 1) to the context
    length, `steps` timed steps after `warmup` untimed ones.  ``model`` may
    be given (configs 4 and 5 share one Mixtral model whose cache is filled
    to 16384 positions; config 4 reads its first 4096); ``sigma``: the
    predictor weights are the model's router + N(0, sigma) copy, None: the
    router itself.  Returns the bench line (a dict), the model and the
    generator."""
    import torch

    from megakernels_amd.mixtral.generate import MK_Generator

    llama = config == "c3"
    if llama:
        from megakernels_amd.latency.synthetic import C3 as cfg
    else:
        from megakernels_amd.mixtral.synthetic import C4 as cfg
    prefill = PREFILL[config]
    if model is None:
        model = build_decode_model(config, prefill + steps + warmup + 1, sigma)
    if not llama and sigma is not None and model.stacked_params.predictor_weight is None:
        raise ValueError("a predictor sigma needs a model built with predictor weights")
    gkw = {"attention_partitions": args.partitions}
    if args.qkv_block:
        gkw["qkv_block_size"] = args.qkv_block
    for kv in args.block_size:
        k, v = kv.split("=", 1)
        gkw[k] = int(v)
    gen = MK_Generator.build(model, prefill, mode=args.assign, globals_kwargs=gkw,
                             dag_kwargs=None if llama else {"predict": not args.no_predict},
                             device_argmax=not args.host_argmax, reset_next=not args.no_reset,
                             late_loads=args.late_loads, xcd_rows=tuple(int(x) for x in args.xcd_rows.split(",") if x),
                             **({} if llama else {"work_sharing": not args.no_work_sharing}))
    if not llama and sigma is None:
        gen.schedule.globs.predictor_weights = None  # opcode 8 predicts with the router itself
    print(f"bench: {config}: {len(gen.schedule.dag_nodes)} instructions per step", file=sys.stderr, flush=True)
    tokens, secs = gen.timed_generate(first_token=1, prompt_len=prefill, ntok=steps, warmup=warmup)
    gpu_s = gen.last_gpu_seconds
    import mk_mixtral

    mk_mixtral.raise_if_failed("cuda")
    print(f"bench: {config} {steps / secs:.1f} tokens/s ({secs / steps * 1e3:.3f} ms per step, "
          f"{gpu_s / steps * 1e3:.3f} ms by HIP events)", file=sys.stderr, flush=True)
    if args.trace:
        from megakernels_amd.trace import TimingRecord, format_report, save_record

        gen.launch_kwargs["record_timings"] = True
        g0 = gen.schedule.globs
        g0.timings.zero_()
        gen.run(tokens[:, -1:], pos_id=prefill + steps)
        torch.cuda.synchronize()
        gen.launch_kwargs.pop("record_timings")
        rec = TimingRecord.from_globals(g0)
        save_record(args.trace, rec)
        print(format_report(rec), file=sys.stderr, flush=True)
    rounds = args.prefetch_ab if prefetch_rounds is None else prefetch_rounds
    ab = prefetch_ab(args, gen, model, prefill, steps, llama, gkw, rounds, sigma) if rounds else None
    ms = secs / steps * 1e3
    nbytes = (decode_bytes_per_token_llama if llama else decode_bytes_per_token)(cfg, prefill + steps // 2)
    kernel_s = gpu_s / steps
    achieved = nbytes / kernel_s / 1e9
    g = gen.schedule.globs
    kernel = "mk_llama_kernel" if llama else "mk_mixtral_kernel<8, true>"
    out = {
        "metric": METRIC,
        "value": steps / secs,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights N(0, 0.02), KV cache N(0, 1))",
        "config": {
            "workload": (f"BASELINE config 3: Llama-3.2-3B-shaped batch-1 greedy decode (28 layers, hidden 3072, "
                         f"24/8 heads, head dim 128, FFN 8192, vocab 128256, RoPE theta 500000), KV cache pre-filled "
                         f"to {prefill} positions, one persistent-kernel launch per token (dense VM)" if llama else
                         f"BASELINE config {'4' if config == 'c4' else '5'}: Mixtral-8x7B-shaped batch-1 greedy "
                         f"decode (32 layers, hidden 4096, 32/8 heads, head dim 128, 8 experts top-2 with FFN 14336, "
                         f"vocab 32000, RoPE theta 1e6), KV cache pre-filled to {prefill} positions, one "
                         f"persistent-kernel launch per token"),
            "prefill": prefill,
            "workers": g.sm_count(),
            "attention_partitions": int(max(i.num_partials for i in gen.schedule.get_linear_instructions()
                                            if i.opcode() == 2)),
            "predictor_sigma": None if llama else sigma,
            "predictor": None if llama else not args.no_predict,
            "assignment": args.assign,
            "qkv_block_size": g.qkv_block_size,
            "block_sizes": {k: getattr(g, k) for k in ("up_gate_proj_block_size", "expert_proj_block_size",
                                                       "down_proj_block_size", "matvec_reduction_size")
                            if hasattr(g, k)},
            "partition_policy": args.partitions,
            "argmax": "torch, between launches" if args.host_argmax else "in-kernel, with the next embedding",
            "late_loads": args.late_loads,
            "work_sharing": None if llama else not args.no_work_sharing,
            "fills_between_launches": args.host_argmax or args.no_reset,
        },
        "ms_per_step_hip_events": kernel_s * 1e3,
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": MEASURED_TRAFFIC_BYTES.get(config),
            "traffic_unit": TRAFFIC_UNIT,
            "bytes_per_launch": nbytes,
            "bytes_per_launch_is": "weights of every layer (attention, norms, router, the two selected experts), "
                                   "K and V of every cached position at the mean context of the timed steps, "
                                   "LM head",
            "kernel": kernel,
            "kernel_time": "HIP events on the launch stream over the timed steps, per step",
        },
        "tokens_tail": tokens[0, -8:].tolist(),
    }
    if ab is not None:
        out["prefetch_ab"] = ab
    return out, model, gen


def prediction_agreement(gen, prefill: int, steps: int = 8) -> dict:
    """Opcode 8's predicted expert pair against the pair opcode 5 selects, in
    every layer of ``steps`` decode steps (timing record on, after the timed
    run; each step's input is the previous step's token): the fraction of
    layers whose predicted top-1 is the selected top-1, whose predicted pair
    is the selected pair as a set (top-2 agreement), and the mean fraction
    of the two selected experts that were predicted."""
    import torch

    from megakernels_amd.trace import T_PREDICTION, TimingRecord

    g = gen.schedule.globs
    gen.launch_kwargs["record_timings"] = True
    tok = torch.ones((1, 1), dtype=torch.long, device=g.hidden_states.device)
    pairs = []
    try:
        for i in range(steps):
            g.timings.zero_()
            tok = gen.run(tok, pos_id=prefill + i).reshape(1, 1)
            torch.cuda.synchronize()
            rec = TimingRecord.from_globals(g)
            ins, tim = rec.instructions, rec.timings
            seen = set()
            for w, q in zip(*((ins[:, :, 0] == 5).nonzero())):
                layer = int(ins[w, q, 1])
                v = int(tim[w, q, T_PREDICTION]) & 0xFFFFFFFF
                if layer in seen or v == 0 or v & 0xFF == 0xFF:
                    continue
                seen.add(layer)
                pairs.append((v & 0xFF, (v >> 8) & 0xFF, (v >> 16) & 0xFF, (v >> 24) & 0xFF))
    finally:
        gen.launch_kwargs.pop("record_timings", None)
        gen.fill()
        gen._clean = False
    n = len(pairs)
    if n == 0:
        return {"layers": 0}
    return {
        "layers": n,
        "steps": steps,
        "top1": sum(p0 == s0 for p0, _, s0, _ in pairs) / n,
        "top2_set": sum({p0, p1} == {s0, s1} for p0, p1, s0, s1 in pairs) / n,
        "expert_overlap": sum(len({p0, p1} & {s0, s1}) for p0, p1, s0, s1 in pairs) / (2 * n),
        "definition": "per layer of each step: predicted top-1 == selected top-1 (top1); predicted pair == "
                      "selected pair as a set (top2_set, the agreement the predictor sigma is tuned for); "
                      "mean fraction of the selected pair that was predicted (expert_overlap)",
    }


def set_predictor_sigma(model, sigma: float, seed: int = 7) -> None:
    """predictor weights <- bf16(router + N(0, sigma)), in place (the
    tensor the launches read)."""
    import torch

    sp = model.stacked_params
    g = torch.Generator(device=sp.router_weight.device)
    g.manual_seed(seed)
    noise = torch.empty(sp.router_weight.shape, dtype=torch.float32, device=sp.router_weight.device)
    noise.normal_(0.0, sigma, generator=g)
    sp.predictor_weight.copy_((sp.router_weight.float() + noise).to(sp.predictor_weight.dtype))


def prefetch_ab(args, gen, model, prefill: int, steps: int, llama: bool, gkw: dict, rounds: int,
                sigma: float | None = None):
    """Prefetch on vs off in the same process, alternating for
    ``args.prefetch_ab`` rounds of ``steps`` decode steps each (medians of
    HIP-event tokens/s): "on" is the default launch; "late_loads" waits for
    every instruction's inputs before any of its loads and stages nothing
    ahead (every early load and all LDS staging off); for the Mixtral shape,
    "no_predict" also leaves out opcode 8 and the predicted-expert staging
    that uses it (the rest of the early loads on).  The reference credits
    its L2 prefetch of next-iteration weights with +5-8 % on Llama-3B
    decode (README.md:13, B200; demos/low-latency-llama/
    matvec_pipeline.cuh:217-233)."""
    import statistics

    import torch

    from megakernels_amd.mixtral.generate import MK_Generator

    base = {"device_argmax": not args.host_argmax, "reset_next": not args.no_reset}
    if not llama:
        base["work_sharing"] = not args.no_work_sharing
    variants = {"on": gen}
    variants["late_loads"] = MK_Generator.build(model, prefill, mode=args.assign, globals_kwargs=gkw,
                                                dag_kwargs=None if llama else {"predict": not args.no_predict},
                                                late_loads=True, **base)
    if not llama:
        variants["no_predict"] = MK_Generator.build(model, prefill, mode=args.assign, globals_kwargs=gkw,
                                                    dag_kwargs={"predict": False}, **base)
        if sigma is None:
            for v in variants.values():
                v.schedule.globs.predictor_weights = None
    rates = {k: [] for k in variants}
    for r in range(rounds):
        for name, g in variants.items():
            g.timed_generate(first_token=1, prompt_len=prefill, ntok=steps, warmup=1)
            rates[name].append(steps / g.last_gpu_seconds)
        print(f"bench: prefetch A/B round {r}: " + ", ".join(f"{k} {v[-1]:.1f}" for k, v in rates.items()),
              file=sys.stderr, flush=True)
    import mk_mixtral

    mk_mixtral.raise_if_failed("cuda")
    med = {k: statistics.median(v) for k, v in rates.items()}
    out = {
        "rounds": rounds,
        "steps_per_round": steps,
        "tokens_per_s": {k: round(v, 2) for k, v in med.items()},
        "all": {k: [round(x, 2) for x in v] for k, v in rates.items()},
        "gain_on_vs_late_loads": med["on"] / med["late_loads"] - 1.0,
        "reference": "+5-8 % from L2 prefetch on Llama-3B decode (README.md:13, NVIDIA B200)",
        "unit": "tokens/s by HIP events, median over rounds",
    }
    if "no_predict" in med:
        out["gain_on_vs_no_predict"] = med["on"] / med["no_predict"] - 1.0
    for name in list(variants):
        if name != "on":
            del variants[name]
    torch.cuda.empty_cache()
    return out


def cpu_baseline_decode(model, prefill: int, seconds: float, threads: int, sm_count: int, layers: int = 2,
                        backend: str = "torch", cpu=None):
    """The CPU oracle (a restatement of the reference's python_vm) on a
    bounded slice of the config-4 decode step: the first ``layers`` layers
    of the same model with the LM head, at the same cached context, stepped
    until ``seconds`` have passed.  ``backend`` "torch": the reference's own
    CPU arithmetic, bf16 einsum per 16-row block and torch CPU attention
    (lat/python_vm.py:29-56); "c": the oracle's C + OpenMP matvecs.  The
    per-layer time and the LM head's time are measured separately and scaled
    to a whole step of all L layers: tokens/s = 1 / (L * t_layer +
    t_lm_head).  Also returns the state after the first step (token 1 at
    position ``prefill``): its token and last-layer experts, for the
    same-run correctness gate."""
    import torch

    from megakernels_amd.mixtral.scheduler import make_dag, make_globals
    from megakernels_amd.mixtral.synthetic import slice_layers
    from megakernels_amd.scheduler import Schedule
    from oracle import python_vm as oracle

    oracle.set_num_threads(threads)
    torch.set_num_threads(threads)
    L = model.config.num_hidden_layers
    if cpu is None:
        cpu = slice_layers(model, layers, "cpu")
    g = make_globals(cpu, seq_len=prefill, sm_count=sm_count)
    g.predictor_weights = None
    g.pos_id = prefill
    nodes, end = make_dag(g)
    linear = Schedule(g, nodes, end).get_linear_instructions()
    t_layers = t_head = 0.0
    steps = 0
    first = None
    oracle.set_backend(backend)
    try:
        t0 = time.perf_counter()
        while steps == 0 or time.perf_counter() - t0 < seconds:
            g.hidden_states.copy_(cpu.embed_tokens[1 + steps])
            g.barriers.zero_()
            g.logits.zero_()
            for ins in linear:
                t1 = time.perf_counter()
                oracle.INSTRUCTION_TO_SOLVER[type(ins)](g, ins)
                dt = time.perf_counter() - t1
                if ins.opcode() == 7:
                    t_head += dt
                else:
                    t_layers += dt
            if steps == 0:
                rl = oracle.router_logits(g.router_weights[layers - 1].contiguous(), g.router_normed_hidden)
                top = torch.sort(rl, descending=True).values
                lg = torch.sort(g.logits.float(), descending=True).values
                first = {"token": int(torch.argmax(g.logits)), "experts": g.selected_expert_indices.tolist(),
                         "router_gaps": [float(top[0] - top[1]), float(top[1] - top[2])],
                         "logit_gap": float(lg[0] - lg[1]), "hidden": g.hidden_states.clone()}
            steps += 1
        elapsed = time.perf_counter() - t0
    finally:
        oracle.set_backend("c")
    per_layer = t_layers / steps / layers
    head = t_head / steps
    token_s = L * per_layer + head
    how = ("bf16 einsum per 16-row block as the reference's python_vm (lat/python_vm.py:29-56), torch CPU "
           "attention" if backend == "torch" else "C+OpenMP matvecs, torch CPU attention")
    out = {
        "value": 1.0 / token_s,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{steps} decode steps of layers 0-{layers - 1} of the same config-4 model with its LM head, "
                  f"{prefill} cached positions, through the oracle python_vm restatement ({len(linear)} "
                  f"instructions per step, {how}), {elapsed:.1f} s; "
                  f"per token = {L} x {per_layer * 1e3:.1f} ms per layer + {head * 1e3:.1f} ms LM head",
        "backend": backend,
        "ms_per_layer": per_layer * 1e3,
        "ms_lm_head": head * 1e3,
        "torch_threads": torch.get_num_threads(),
        "cpu_model": cpu_model_name(),
        "os_cpu_count": os.cpu_count(),
    }
    return out, first


#: router-logit / LM-head logit gap below which the gate accepts a
#: different order (after two layers the residual differs from the
#: oracle's by up to max-abs-rel ~1e-2)
GATE_MARGIN = 0.05


def decode_gate(model, prefill: int, oracle_first: dict, sm_count: int, layers: int = 2) -> dict:
    """Same-run correctness gate of the headline: one launch of the
    whole-model kernel over the same ``layers``-layer slice of the model
    (its LM head included) that the CPU oracle stepped, from the same token
    and position; the token (argmax inside the launch) and the last layer's
    expert pair against the oracle's, exact unless the oracle's own gap is
    below GATE_MARGIN, and the residual within max-abs-rel 2e-2."""
    import torch

    import mk_mixtral
    from megakernels_amd.mixtral.mk import interpret_with_mk
    from megakernels_amd.mixtral.scheduler import make_dag, make_globals
    from megakernels_amd.mixtral.synthetic import slice_layers
    from megakernels_amd.scheduler import Schedule, assign_to_sms, tensorize_instructions

    sl = slice_layers(model, layers, "cuda")
    g = make_globals(sl, seq_len=prefill, sm_count=sm_count)
    g.predictor_weights = None
    g.pos_id = prefill
    nodes, end = make_dag(g)
    tensorize_instructions(g, assign_to_sms("rr", schedule=Schedule(g, nodes, end)))
    g.hidden_states.copy_(sl.embed_tokens[1])
    g.barriers.zero_()
    g.logits.zero_()
    tok = torch.full((), -1, dtype=torch.long, device="cuda")
    interpret_with_mk(g, mk_mixtral.mk_mixtral, argmax_out=tok, debug_sync=True, work_sharing=True)
    torch.cuda.synchronize()
    gtok, gexp = int(tok), g.selected_expert_indices.cpu().tolist()
    ref = oracle_first
    gap01, gap12 = ref["router_gaps"]
    if gap12 < GATE_MARGIN:
        experts_ok = gexp[0] == ref["experts"][0] or gap01 < GATE_MARGIN
    elif gap01 < GATE_MARGIN:
        experts_ok = sorted(gexp) == sorted(ref["experts"])
    else:
        experts_ok = gexp == ref["experts"]
    token_ok = gtok == ref["token"] or ref["logit_gap"] < GATE_MARGIN
    h, r = g.hidden_states.cpu().float(), ref["hidden"].float()
    err = float((h - r).abs().max() / r.abs().max())
    del sl, g
    torch.cuda.empty_cache()
    return {
        "what": f"one whole-model launch over layers 0-{layers - 1} of the bench model with its LM head (token 1 "
                f"at position {prefill}) against the CPU oracle's first step of the same slice",
        "token": gtok, "oracle_token": ref["token"], "oracle_logit_gap": ref["logit_gap"],
        "last_layer_experts": gexp, "oracle_experts": ref["experts"], "oracle_router_gaps": ref["router_gaps"],
        "hidden_max_abs_rel": err,
        "passed": bool(token_ok and experts_ok and err <= 2e-2),
    }


def c2_gate(bench, n: int = 8) -> dict:
    """Same-run correctness gate of the config-2 layer: ``n`` of its tokens
    launched one by one and run through the CPU oracle (C backend) from the
    same residuals; expert pairs exact, hidden and SiLU within max-abs-rel
    2e-2 (drawn residuals: where the oracle's 2nd and 3rd router logits are
    within 1e-3, the order of the pair is not held)."""
    import torch

    from megakernels_amd.mixtral.scheduler import make_globals, prefill_oproj_barrier
    from megakernels_amd.mixtral.synthetic import to_device
    from oracle import python_vm as oracle

    cpu_model = to_device(bench.model, "cpu")
    g = make_globals(cpu_model, sm_count=bench.globs.sm_count(),
                     expert_proj_block_size=bench.globs.expert_proj_block_size,
                     down_proj_block_size=bench.globs.down_proj_block_size)
    linear = bench.linear_instructions()
    residuals = bench.residuals.cpu()
    stream = ctypes.c_void_p(torch.cuda.current_stream(bench.dev).cuda_stream)
    equal = ties = 0
    worst = 0.0
    for t in range(n):
        bench.work[t].copy_(bench.residuals[t])
        bench.bars[t].copy_(bench.bars_init[t])
        bench._launch(t, stream)
        torch.cuda.synchronize()
        gi = bench.globs.selected_expert_indices.cpu()
        silu = bench.globs.expert_silu_out.cpu()
        gh = bench.work[t].cpu()
        g.barriers.zero_()
        prefill_oproj_barrier(g)
        g.hidden_states.copy_(residuals[t])
        oracle.interpret_with_pyvm(g, linear)
        ri = g.selected_expert_indices
        rl = torch.sort(oracle.router_logits(g.router_weights[0].contiguous(), g.router_normed_hidden),
                        descending=True).values
        if torch.equal(gi, ri):
            equal += 1
        elif float(rl[1] - rl[2]) < 1e-3 or float(rl[0] - rl[1]) < 1e-3:
            ties += 1
        idx = ri.long()
        for y, r in ((gh, g.hidden_states), (silu[idx], g.expert_silu_out[idx])):
            worst = max(worst, float((y.float() - r.float()).abs().max() / r.float().abs().max()))
    bench.check_status()
    return {"tokens": n, "experts_equal": equal, "near_ties": ties, "max_abs_rel_hidden_silu": worst,
            "passed": equal + ties == n and worst <= 2e-2}


def layer_bench(args, config: str, steps: int, warmup: int):
    """One MoE layer per launch (config 2 or 1), uniform and skewed; returns
    the figures and the uniform bench object."""
    import torch

    from megakernels_amd.mixtral.synthetic import C1, C2

    cfg = C2 if config == "c2" else C1
    print(f"bench: building {config} weights and {args.tokens} tokens on cuda:0", file=sys.stderr, flush=True)
    overlap = args.moe_overlap
    bal = tuple(int(x) for x in args.balance_opcodes.split(","))
    bench = MoEBench(cfg, args.tokens, seed=0, work_sharing=args.work_sharing, balance=args.balance,
                     moe_overlap=overlap, upgate_rounds=args.upgate_rounds, balance_opcodes=bal)
    timed = run_timed(bench, steps, warmup)
    dist = bench.per_launch_us(256)
    if args.trace and config != "c4":
        record_trace(bench, args.trace)
    nbytes = moe_layer_bytes(cfg)
    us = timed["us_per_launch_events"]
    achieved = nbytes / (us * 1e-6) / 1e9
    print(f"bench: {config} uniform {us:.2f} us/launch, {achieved:.0f} GB/s", file=sys.stderr, flush=True)
    skewed = None
    if not args.no_skewed:
        sk = MoEBench(cfg, args.tokens, seed=0, work_sharing=args.work_sharing, balance=args.balance,
                      moe_overlap=overlap, upgate_rounds=args.upgate_rounds, balance_opcodes=bal,
                      router_bias=[2.0, 2.0] + [0.0] * (cfg.num_local_experts - 2))
        sk_timed = run_timed(sk, max(1, steps // 2), 1)
        sk_us = sk_timed["us_per_launch_events"]
        skewed = {"moe_layer_us": sk_us, "hbm_frac": nbytes / (sk_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
                  "router_bias": "+2.0 on experts 0 and 1"}
        del sk
        torch.cuda.empty_cache()
        print(f"bench: {config} skewed {sk_us:.2f} us/launch", file=sys.stderr, flush=True)
    g = bench.globs
    fig = {
        "workload": f"BASELINE config {'2' if config == 'c2' else '1'}: one Mixtral-8x7B-shaped MoE layer (hidden "
                    f"{cfg.hidden_size}, FFN {cfg.intermediate_size}, {cfg.num_local_experts} experts, "
                    f"top-{cfg.num_experts_per_tok}), {bench.tokens} batch-1 tokens per step with residuals N(0, 1), "
                    "one persistent-kernel launch (opcodes 5 and 6) per token",
        "steps": steps,
        "ms_per_step": timed["wall_s"] / steps * 1e3,
        "tokens_per_step": bench.tokens,
        "workers": g.sm_count(),
        "expert_proj_block_size": g.expert_proj_block_size,
        "down_proj_block_size": g.down_proj_block_size,
        "work_sharing": args.work_sharing,
        "speed_balanced_partition": args.balance,
        "moe_overlap": overlap,
        "moe_layer_us": us,
        "moe_layer_us_per_launch": dist,
        "hbm_frac": achieved / HBM_PEAK_GBS,
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": MEASURED_TRAFFIC_BYTES.get(config),
            "traffic_unit": TRAFFIC_UNIT,
            "bytes_per_launch": nbytes,
            "kernel": "mk_mixtral_kernel<8, false>",
            "kernel_time": "HIP events on the launch stream over the timed steps, per launch",
        },
        "skewed": skewed,
    }
    return fig, bench, timed


def cpu_baseline_layer(bench, seconds: float, threads: int):
    """The CPU oracle (restated python_vm, C + OpenMP) on the same weights,
    inputs and instruction list as the MoE-layer bench, over a bounded sample
    of tokens."""
    import torch

    from megakernels_amd.mixtral.scheduler import make_globals, prefill_oproj_barrier
    from megakernels_amd.mixtral.synthetic import to_device
    from oracle import python_vm as oracle

    oracle.set_num_threads(threads)
    cpu_model = to_device(bench.model, "cpu")
    g = make_globals(cpu_model, sm_count=bench.globs.sm_count(),
                     expert_proj_block_size=bench.globs.expert_proj_block_size,
                     down_proj_block_size=bench.globs.down_proj_block_size)
    linear = bench.linear_instructions()
    residuals = bench.residuals.cpu()
    done = 0
    agree = 0
    t0 = time.perf_counter()
    while done < bench.tokens and (done == 0 or time.perf_counter() - t0 < seconds):
        g.barriers.zero_()
        prefill_oproj_barrier(g)
        g.hidden_states.copy_(residuals[done])
        oracle.interpret_with_pyvm(g, linear)
        done += 1
    elapsed = time.perf_counter() - t0
    # selection parity of the sampled tokens against the kernel
    for t in range(done):
        bench.work[t].copy_(bench.residuals[t])
        bench.bars[t].copy_(bench.bars_init[t])
    stream = ctypes.c_void_p(torch.cuda.current_stream(bench.dev).cuda_stream)
    sel = []
    for t in range(done):
        bench._launch(t, stream)
        sel.append(bench.globs.selected_expert_indices.clone())
    torch.cuda.synchronize()
    for t in range(done):
        g.barriers.zero_()
        prefill_oproj_barrier(g)
        g.hidden_states.copy_(residuals[t])
        oracle.interpret_with_pyvm(g, linear)
        agree += int(torch.equal(sel[t].cpu(), g.selected_expert_indices))
    return {
        "value": done / elapsed,
        "unit": "MoE-layer tokens/s",
        "cores": oracle.get_num_threads(),
        "kind": "port",
        "sample": f"{done} config-2 tokens through the oracle python_vm restatement (opcodes 5+6, "
                  f"{len(linear)} instructions each, C+OpenMP), {elapsed:.1f} s",
        "moe_layer_us": elapsed / done * 1e6,
        "cpu_model": cpu_model_name(),
        "os_cpu_count": os.cpu_count(),
        "selection_agrees_with_gpu": f"{agree}/{done}",
    }


def compact(line: dict) -> dict:
    """The figures of a decode bench line that another config's line carries."""
    keep = ("value", "unit", "steps", "warmup", "ms_per_step", "ms_per_step_hip_events", "roofline", "prefetch_ab",
            "prediction_agreement", "tokens_tail")
    out = {k: line[k] for k in keep if k in line}
    out["config"] = line["config"]
    return out


def headline(args, threads: int, warmup: int) -> dict:
    """The default run.  Config 4 is the headline (``value``); configs 2, 5
    and 3 are timed in the same process and carried as extra keys, each with
    its own roofline:

    1. config 2 (one MoE layer per launch) on the fresh device, with its
       same-run correctness gate;
    2. one Mixtral model whose KV cache is filled to 16384 positions:
       config 4 decodes at 4096 (predictor = the router), then the CPU
       oracle on a two-layer slice of it (torch-bf16 and C legs) and the
       same-run correctness gate, then config 5 at 16384 with predictor
       weights = router + N(0, C5_SIGMA), its predictor A/B and the
       measured prediction agreement;
    3. config 3 (Llama-3.2-3B shape, dense VM) on its own model."""
    import torch

    layer_fig = None
    if not args.no_layer:
        layer_fig, bench, _ = layer_bench(args, "c2", args.layer_steps, 2)
        layer_fig["correctness"] = c2_gate(bench)
        print(f"bench: c2 gate {layer_fig['correctness']}", file=sys.stderr, flush=True)
        del bench
        torch.cuda.empty_cache()
    steps = args.steps or args.decode_steps or 128
    c5_steps = args.extra_steps or 128
    sigma = C5_SIGMA if args.predict_sigma is None else args.predict_sigma
    positions = PREFILL["c5"] + max(steps + warmup, c5_steps + 2, 8) + 16
    model = build_decode_model("c4", positions, sigma, prefill=PREFILL["c5"])
    out, model, gen = decode_bench(args, "c4", steps, warmup, model=model, sigma=None)
    sm = gen.schedule.globs.sm_count()
    del gen
    if not args.no_cpu:
        print(f"bench: CPU oracle baseline ({threads} threads, ~{args.cpu_seconds:.0f} s per leg)", file=sys.stderr,
              flush=True)
        cpu_t, first = cpu_baseline_decode(model, PREFILL["c4"], args.cpu_seconds, threads, sm, backend="torch")
        cpu_c, _ = cpu_baseline_decode(model, PREFILL["c4"], args.cpu_seconds, threads, sm, backend="c")
        cpu_t["c_openmp_leg"] = cpu_c
        out["cpu_baseline"] = cpu_t
        out["correctness"] = decode_gate(model, PREFILL["c4"], first, sm)
        print(f"bench: c4 gate passed={out['correctness']['passed']}", file=sys.stderr, flush=True)
    extra = {}
    args.trace = ""  # a --trace record is of the headline (config 4) step
    if not args.no_extra:
        c5, model, gen = decode_bench(args, "c5", c5_steps, 2, model=model, sigma=sigma)
        c5["prediction_agreement"] = prediction_agreement(gen, PREFILL["c5"])
        print(f"bench: c5 prediction agreement {c5['prediction_agreement']}", file=sys.stderr, flush=True)
        extra["c5"] = compact(c5)
        del gen
    del model
    torch.cuda.empty_cache()
    if not args.no_extra:
        c3_steps = args.extra_steps or 256
        c3, m3, gen = decode_bench(args, "c3", c3_steps, 2)
        extra["c3"] = compact(c3)
        del m3, gen
        torch.cuda.empty_cache()
    if layer_fig is not None:
        out["moe_layer"] = layer_fig
    if extra:
        out["configs"] = extra
    return out


def sigma_sweep(args, model, sigmas) -> list:
    """Prediction agreement of the config-5 decode (16384 cached positions)
    for each predictor noise level: predictor weights <- router + N(0,
    sigma), then the agreement over 8 recorded steps of all layers."""
    from megakernels_amd.mixtral.generate import MK_Generator

    gen = MK_Generator.build(model, PREFILL["c5"], mode=args.assign,
                             globals_kwargs={"attention_partitions": args.partitions})
    out = []
    for sg in sigmas:
        set_predictor_sigma(model, sg)
        a = prediction_agreement(gen, PREFILL["c5"])
        a["sigma"] = sg
        print(f"bench: sigma {sg}: {a}", file=sys.stderr, flush=True)
        out.append(a)
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=0,
                    help="timed steps (default: 128 decode steps for c4/c5, 256 for c3 as BASELINE states them; "
                         "10 steps of --tokens launches for c1/c2)")
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--tokens", type=int, default=1024, help="c1/c2 (and the headline's layer figures): tokens "
                                                             "per step")
    ap.add_argument("--config", default="c4", choices=["c1", "c2", "c3", "c4", "c5"],
                    help="c4 (default): whole-model greedy decode of the Mixtral-8x7B shape with 4096 cached "
                         "positions, plus the config-2 MoE layer figures and the CPU baseline; c5: the same with "
                         "16384 cached positions; c3: the Llama-3.2-3B shape (2048 cached positions, dense VM); "
                         "c1/c2: one MoE layer per launch alone")
    ap.add_argument("--decode-steps", type=int, default=0, help="alias of --steps for c3/c4/c5")
    ap.add_argument("--layer-steps", type=int, default=10,
                    help="c4: timed steps (of --tokens launches) of the config-2 layer figures")
    ap.add_argument("--no-layer", action="store_true", help="c4: leave out the config-2 layer figures")
    ap.add_argument("--c4-only", action="store_true",
                    help="c4: the config-4 decode alone (with its CPU baseline and gate), not the default line "
                         "that also times configs 2, 5 and 3")
    ap.add_argument("--no-extra", action="store_true", help="default run: leave out configs 5 and 3")
    ap.add_argument("--extra-steps", type=int, default=0,
                    help="default run: timed steps of configs 5 and 3 (default: 128 and 256, as BASELINE states)")
    ap.add_argument("--sigma-sweep", default="", metavar="S1,S2,...",
                    help="c5: only measure the prediction agreement for each predictor noise level and exit")
    ap.add_argument("--assign", default="rr", choices=["rr", "zz", "wave", "dag"],
                    help="c3/c4/c5: instruction-to-worker assignment of the whole-model schedule")
    ap.add_argument("--qkv-block", type=int, default=0,
                    help="c3/c4/c5: QKV row block size (default: picked for the worker count)")
    ap.add_argument("--partitions", default="mi355x",
                    help="c3/c4/c5: split-KV partition policy: mi355x, mi355x:N (at most N partitions per KV head) "
                         "or reference")
    ap.add_argument("--block-size", action="append", default=[], metavar="NAME=N",
                    help="c3/c4/c5: override a block size of make_globals (e.g. up_gate_proj_block_size, "
                         "down_proj_block_size, o_proj_block_size, lm_head_block_size, matvec_reduction_size)")
    ap.add_argument("--no-predict", action="store_true",
                    help="c4/c5: leave out opcode 8 (expert prediction) and the early expert loads that use it")
    ap.add_argument("--predict-sigma", type=float, default=None,
                    help="c5: predictor weights = router + N(0, sigma) (default: C5_SIGMA; config 4 predicts "
                         "with the router itself)")
    ap.add_argument("--late-loads", action="store_true",
                    help="c3/c4/c5: prefetch off -- every instruction waits for its inputs before any of its "
                         "loads, nothing is staged ahead in LDS")
    ap.add_argument("--prefetch-ab", type=int, default=3, metavar="ROUNDS",
                    help="c3/c4/c5: after the timed run, ROUNDS alternating rounds of prefetch on / late loads "
                         "(/ no predictor, Mixtral) in the same process, reported as prefetch_ab (0: skip)")
    ap.add_argument("--host-argmax", action="store_true",
                    help="c3/c4/c5: torch.argmax and the embedding lookup between launches, as the reference's "
                         "generator (default: inside the launch)")
    ap.add_argument("--no-reset", action="store_true",
                    help="c3/c4/c5: fill the barriers and logits before every launch instead of having each "
                         "launch zero them for the next")
    ap.add_argument("--xcd-rows", default="", metavar="OPCODES",
                    help="c3/c4/c5: comma-separated opcodes whose row ranges are regrouped so each XCD's workers "
                         "take one contiguous span (group_rows_by_xcd)")
    ap.add_argument("--no-skewed", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-threads", type=int, default=int(os.environ.get("OMP_NUM_THREADS", "0") or 0))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--moe-overlap", choices=["on", "off", "op5", "op6"], default="off",
                    help="c1/c2: interleaved opcode-5 partition with opcode 6 starting on finished SiLU "
                         "column groups (on), the reference's contiguous partition and full barrier (off), "
                         "or one half alone: the interleaved partition with the full barrier (op5), the "
                         "grouped opcode 6 on the contiguous partition (op6)")
    ap.add_argument("--upgate-rounds", type=int, default=3,
                    help="c1/c2 with --moe-overlap on/op5: contiguous opcode-5 block runs per worker")
    ap.add_argument("--balance-opcodes", default="5,6",
                    help="with --balance: the opcodes whose rows are re-split by measured speed")
    ap.add_argument("--balance", action="store_true",
                    help="re-split rows by per-worker speed measured on a few launches (block size 1)")
    ap.add_argument("--work-sharing", action="store_true",
                    help="c1/c2: idle workers take unclaimed opcode-5 rows of other workers (c4/c5: the default)")
    ap.add_argument("--no-work-sharing", action="store_true",
                    help="c4/c5: every worker does exactly its own opcode-5 rows")
    ap.add_argument("--trace", default="", metavar="NPZ",
                    help="after the timed run, record the kernel's timing slots (8 launches for c1/c2, one decode "
                         "step for c3/c4/c5), save the last as NPZ and print the trace analysis to stderr")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 device-to-device copies of MIB MiB (reads MIB, writes MIB) and exit; "
                         "the known-size kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the expert/tensor-parallel split is a design, not a benchmarked path", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "launches": 5}), flush=True)
        return

    threads = args.cpu_threads or os.cpu_count()
    warmup = max(1, args.warmup)
    if args.config in ("c3", "c4", "c5"):
        if args.config == "c4" and not args.c4_only:
            print(json.dumps(headline(args, threads, warmup)), flush=True)
            return
        steps = args.steps or args.decode_steps or (256 if args.config == "c3" else 128)
        sigma = args.predict_sigma
        if sigma is None and args.config == "c5":
            sigma = C5_SIGMA
        model = None
        if args.config != "c3":
            positions = PREFILL[args.config] + steps + warmup + 16
            model = build_decode_model(args.config, positions, sigma)
            if args.sigma_sweep:
                sweep = sigma_sweep(args, model, [float(x) for x in args.sigma_sweep.split(",")])
                print(json.dumps({"sigma_sweep": sweep}), flush=True)
                return
        out, model, gen = decode_bench(args, args.config, steps, warmup, model=model, sigma=sigma)
        if args.config == "c5":
            out["prediction_agreement"] = prediction_agreement(gen, PREFILL["c5"])
        if args.config == "c4" and not args.no_cpu:
            out["cpu_baseline"], first = cpu_baseline_decode(model, PREFILL["c4"], args.cpu_seconds, threads,
                                                             gen.schedule.globs.sm_count())
            out["correctness"] = decode_gate(model, PREFILL["c4"], first, gen.schedule.globs.sm_count())
        del model, gen
        torch.cuda.empty_cache()
        print(json.dumps(out), flush=True)
        return

    steps = args.steps or 10
    fig, bench, timed = layer_bench(args, args.config, steps, args.warmup)
    cpu = None
    if not args.no_cpu:
        print(f"bench: CPU oracle baseline ({threads} threads, ~{args.cpu_seconds:.0f} s)", file=sys.stderr,
              flush=True)
        cpu = cpu_baseline_layer(bench, args.cpu_seconds, threads)
    out = {
        "metric": METRIC,
        "value": bench.tokens * steps / timed["wall_s"],
        "unit": "MoE-layer tokens/s (one layer per launch, not whole-model decode)",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": timed["wall_s"] / steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights N(0, 0.02), residuals N(0, 1))",
        "config": {k: fig[k] for k in ("workload", "tokens_per_step", "workers", "expert_proj_block_size",
                                       "down_proj_block_size", "work_sharing", "speed_balanced_partition",
                                       "moe_overlap")},
        "moe_layer_us": fig["moe_layer_us"],
        "moe_layer_us_per_launch": fig["moe_layer_us_per_launch"],
        "hbm_frac": fig["hbm_frac"],
        "roofline": fig["roofline"],
        "skewed": fig["skewed"],
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
