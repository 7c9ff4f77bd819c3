"""Whole-model decode steps on the GPU (all opcodes, 1-8) and on the CPU
oracle PyVM, from the same weights, KV cache and instruction list.

A step follows the reference's generator (megakernels/generators.py:121-146):
hidden <- embedding of the input token, barriers and logits zeroed, pos_id
set, one launch over the whole-model schedule.  Both sides then advance by
one position: the GPU kernel appends K/V at pos_id, as does the oracle.
"""

from __future__ import annotations

import torch

from megakernels_amd.mixtral.scheduler import make_dag, make_globals
from megakernels_amd.mixtral.synthetic import make_synthetic_mixtral, to_device
from megakernels_amd.scheduler import Schedule, assign_to_sms, tensorize_instructions
from moe_harness import max_abs_rel
from oracle import python_vm as oracle


class FullCase:
    def __init__(self, config, seed=0, prefill=20, steps=4, workers=None, mode="rr", ln_weight_std=0.1,
                 stop_after_op=None, layer_limit=None):
        cpu = make_synthetic_mixtral(config, "cpu", seed, full=True, kv_positions=prefill + steps + 1,
                                     prefill=prefill, ln_weight_std=ln_weight_std)
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
        import mk_mixtral
        from megakernels_amd.mixtral.mk import interpret_with_mk

        for g, model in ((self.g_cpu, self.cpu_model), (self.g_gpu, self.gpu_model)):
            g.hidden_states.copy_(model.embed_tokens[token])
            g.barriers.zero_()
            g.logits.zero_()
            g.pos_id = self.pos
        kw.setdefault("debug_sync", True)
        interpret_with_mk(self.g_gpu, mk_mixtral.mk_mixtral, **kw)
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
        if r.logits.any():
            err["logits"] = max_abs_rel(g.logits, r.logits)
        return err

    def barriers_equal(self) -> bool:
        return torch.equal(self.g_gpu.barriers.cpu(), self.g_cpu.barriers)

    def indices(self):
        return self.g_gpu.selected_expert_indices.cpu().tolist(), self.g_cpu.selected_expert_indices.tolist()
