"""Whole-model decode steps of the dense (Llama) VM on the GPU and on the
CPU oracle (oracle/latency_vm.py), from the same weights, KV cache and
instruction list; a step follows megakernels/generators.py:121-146."""

from __future__ import annotations

import torch

from megakernels_amd.latency.scheduler import make_dag, make_globals
from megakernels_amd.latency.synthetic import make_synthetic_llama, to_device
from megakernels_amd.scheduler import Schedule, assign_to_sms, tensorize_instructions
from moe_harness import max_abs_rel
from oracle import latency_vm as oracle


class LlamaCase:
    def __init__(self, config, seed=0, prefill=20, steps=4, workers=None, mode="rr", ln_weight_std=0.1,
                 stop_after_op=None, layer_limit=None):
        cpu = make_synthetic_llama(config, "cpu", seed, ln_weight_std=ln_weight_std,
                                   kv_positions=prefill + steps + 1, prefill=prefill)
        self.cpu_model = cpu
        self.gpu_model = to_device(cpu, "cuda")
        if workers is None:
            workers = torch.cuda.get_device_properties(0).multi_processor_count
        self.g_cpu = make_globals(self.cpu_model, sm_count=workers, seq_len=prefill)
        self.g_gpu = make_globals(self.gpu_model, sm_count=workers, seq_len=prefill)
        self.g_gpu.pos_id = self.g_cpu.pos_id = prefill
        nodes, end = make_dag(self.g_gpu, stop_after_op=stop_after_op, layer_limit=layer_limit)
        self.schedule = Schedule(self.g_gpu, nodes, end)
        self.g_cpu.skip_attn_reduction = self.g_gpu.skip_attn_reduction
        tensorize_instructions(self.g_gpu, assign_to_sms(mode, schedule=self.schedule))
        self.linear = self.schedule.get_linear_instructions()
        self.pos = prefill

    def step(self, token: int, **kw):
        import mk_llama
        from megakernels_amd.latency.mk import interpret_with_mk

        for g, model in ((self.g_cpu, self.cpu_model), (self.g_gpu, self.gpu_model)):
            g.hidden_states.copy_(model.embed_tokens[token])
            g.barriers.zero_()
            g.logits.zero_()
            g.pos_id = self.pos
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

    def barriers_equal(self) -> bool:
        return torch.equal(self.g_gpu.barriers.cpu(), self.g_cpu.barriers)
