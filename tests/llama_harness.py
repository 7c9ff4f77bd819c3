"""Whole-model decode steps of the dense (Llama) VM on the GPU and on the
CPU oracle (oracle/latency_vm.py), from the same weights, KV cache and
instruction list; a step follows megakernels/generators.py:121-146.

``start_after_op`` runs the schedule's prefix up to that stage of layer 0 on
the oracle and hands its state to the kernel, as ``full_harness.FullCase``
does (megakernels/scripts/diff_test.py:139-162)."""

from __future__ import annotations

import torch

from full_harness import copy_state, split_linear
from megakernels_amd.latency.scheduler import make_dag, make_globals
from megakernels_amd.latency.synthetic import make_synthetic_llama, to_device
from megakernels_amd.scheduler import Schedule, assign_to_sms, tensorize_instructions
from moe_harness import bf16_agreement, max_abs_rel
from oracle import latency_vm as oracle

MUTABLE = ("hidden_states", "post_ln_rope_q", "attn_out", "attn_out_intermediates", "attn_lse_intermediates",
           "silu_out", "logits", "barriers", "k_cache", "v_cache")


class LlamaCase:
    def __init__(self, config, seed=0, prefill=20, steps=4, workers=None, mode="rr", ln_weight_std=0.1,
                 stop_after_op=None, layer_limit=None, start_after_op=None, generate_on_device=False, **globals_kw):
        kv = prefill + steps + 1
        if generate_on_device:
            gpu = make_synthetic_llama(config, "cuda", seed, ln_weight_std=ln_weight_std, kv_positions=kv,
                                       prefill=prefill)
            self.gpu_model, self.cpu_model = gpu, to_device(gpu, "cpu")
        else:
            cpu = make_synthetic_llama(config, "cpu", seed, ln_weight_std=ln_weight_std, kv_positions=kv,
                                       prefill=prefill)
            self.cpu_model, self.gpu_model = cpu, to_device(cpu, "cuda")
        if workers is None:
            workers = torch.cuda.get_device_properties(0).multi_processor_count
        self.g_cpu = make_globals(self.cpu_model, sm_count=workers, seq_len=prefill, **globals_kw)
        self.g_gpu = make_globals(self.gpu_model, sm_count=workers, seq_len=prefill, **globals_kw)
        self.g_gpu.pos_id = self.g_cpu.pos_id = prefill
        if start_after_op is None:
            nodes, end = make_dag(self.g_gpu, stop_after_op=stop_after_op, layer_limit=layer_limit)
            self.schedule = Schedule(self.g_gpu, nodes, end)
            self.prefix = []
            self.linear = self.schedule.get_linear_instructions()
            queues = assign_to_sms(mode, schedule=self.schedule)
        else:
            self.prefix, self.linear = split_linear(make_dag, self.g_gpu, start_after_op, layer_limit, stop_after_op)
            assert mode in ("rr", "zz"), "a schedule suffix is assigned from its instruction list"
            queues = assign_to_sms(mode, instructions=self.linear, sm_count=workers)
        self.g_cpu.skip_attn_reduction = self.g_gpu.skip_attn_reduction
        tensorize_instructions(self.g_gpu, queues)
        self.pos = prefill

    def step(self, token: int, **kw):
        import mk_llama
        from megakernels_amd.latency.mk import interpret_with_mk

        for g, model in ((self.g_cpu, self.cpu_model), (self.g_gpu, self.gpu_model)):
            g.hidden_states.copy_(model.embed_tokens[token])
            g.barriers.zero_()
            g.logits.zero_()
            g.pos_id = self.pos
        if self.prefix:
            oracle.interpret_with_pyvm(self.g_cpu, self.prefix)
            copy_state(self.g_gpu, self.g_cpu, MUTABLE)
        kw.setdefault("debug_sync", True)
        interpret_with_mk(self.g_gpu, mk_llama.mk_llama, **kw)
        torch.cuda.synchronize()
        oracle.interpret_with_pyvm(self.g_cpu, self.linear)
        self.pos += 1

    def errors(self) -> dict:
        g, r = self.g_gpu, self.g_cpu
        pos = self.pos - 1
        err = {
            "hidden": max_abs_rel(g.hidden_states, r.hidden_states),
            "k_new": max_abs_rel(g.k_cache[:, 0, pos], r.k_cache[:, 0, pos]),
            "v_new": max_abs_rel(g.v_cache[:, 0, pos], r.v_cache[:, 0, pos]),
            "q": max_abs_rel(g.post_ln_rope_q, r.post_ln_rope_q),
            "attn_out": max_abs_rel(g.attn_out, r.attn_out),
        }
        if r.silu_out.any():
            err["silu"] = max_abs_rel(g.silu_out, r.silu_out)
        if r.logits.any():
            err["logits"] = max_abs_rel(g.logits, r.logits)
        return err

    def agreement(self) -> dict:
        """(max bf16 ulps, bit-identical fraction) against the oracle."""
        g, r = self.g_gpu, self.g_cpu
        pos = self.pos - 1
        out = {
            "hidden": bf16_agreement(g.hidden_states, r.hidden_states),
            "k_new": bf16_agreement(g.k_cache[:, 0, pos], r.k_cache[:, 0, pos]),
            "v_new": bf16_agreement(g.v_cache[:, 0, pos], r.v_cache[:, 0, pos]),
            "q": bf16_agreement(g.post_ln_rope_q, r.post_ln_rope_q),
            "attn_out": bf16_agreement(g.attn_out, r.attn_out),
        }
        if r.silu_out.any():
            out["silu"] = bf16_agreement(g.silu_out, r.silu_out)
        if r.logits.any():
            out["logits"] = bf16_agreement(g.logits, r.logits)
        return out

    def barriers_equal(self) -> bool:
        return torch.equal(self.g_gpu.barriers.cpu(), self.g_cpu.barriers)
