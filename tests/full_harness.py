"""Whole-model decode steps on the GPU (all opcodes, 1-8) and on the CPU
oracle PyVM, from the same weights, KV cache and instruction list.

A step follows the reference's generator (megakernels/generators.py:121-146):
hidden <- embedding of the input token, barriers and logits zeroed, pos_id
set, one launch over the whole-model schedule.  Both sides then advance by
one position: the GPU kernel appends K/V at pos_id, as does the oracle.

``start_after_op`` is the reference diff harness's stage mode
(megakernels/scripts/diff_test.py:139-162, 214-224): the schedule's prefix up
to and including that stage of layer 0 runs on the oracle, the state it
leaves (activations, intermediates, K/V rows, barriers) is copied to the GPU,
and the rest of the schedule runs on the kernel and on the oracle from that
same state.  With ``stop_after_op`` as well, the rest is just the stages
between the two, so one stage can be run alone from bit-identical inputs and
its rounding points checked with no drift from earlier stages.

Large shapes (``generate_on_device=True``) draw the weights on the GPU and
copy them to the host for the oracle: the same tensors on both sides, drawn
in seconds instead of minutes.
"""

from __future__ import annotations

import torch

from megakernels_amd.mixtral.scheduler import make_dag, make_globals
from megakernels_amd.mixtral.synthetic import make_synthetic_mixtral, to_device
from megakernels_amd.scheduler import Schedule, assign_to_sms, tensorize_instructions
from moe_harness import bf16_agreement, max_abs_rel
from oracle import python_vm as oracle

#: tensors of MixtralGlobals that a launch writes (the state a prefix hands on)
MUTABLE = ("hidden_states", "post_ln_rope_q", "attn_out", "attn_out_intermediates", "attn_lse_intermediates",
           "expert_silu_out", "router_normed_hidden", "logits", "selected_expert_indices",
           "selected_expert_scores", "predicted_expert_indices", "barriers", "k_cache", "v_cache")


def split_linear(dag_fn, globs, start_after_op: str, layer_limit: int | None, stop_after_op: str | None = None,
                 **dag_kw):
    """(prefix, suffix) of the linear instruction list of ``dag_fn(globs,
    stop_after_op=stop_after_op, layer_limit=layer_limit)``: the prefix is
    the schedule that stops after ``start_after_op`` in layer 0, which must
    be a prefix of the whole (megakernels/scripts/diff_test.py:139-153).
    With both, the suffix is the stages between the two."""
    nodes, end = dag_fn(globs, stop_after_op=stop_after_op, layer_limit=layer_limit, **dag_kw)
    full = Schedule(globs, nodes, end).get_linear_instructions()
    pnodes, pend = dag_fn(globs, stop_after_op=start_after_op, layer_limit=1, **dag_kw)
    prefix = Schedule(globs, pnodes, pend).get_linear_instructions()
    assert len(prefix) < len(full), f"prefix of {len(prefix)} is not shorter than the {len(full)} instructions"
    for a, b in zip(prefix, full):
        assert a == b, f"{a} is not a prefix instruction of the whole schedule"
    return prefix, full[len(prefix):]


def copy_state(dst, src, names=MUTABLE):
    for n in names:
        getattr(dst, n).copy_(getattr(src, n).to(getattr(dst, n).device))


class FullCase:
    def __init__(self, config, seed=0, prefill=20, steps=4, workers=None, mode="rr", ln_weight_std=0.1,
                 stop_after_op=None, layer_limit=None, start_after_op=None, generate_on_device=False,
                 predictor_sigma=None, predict=True, **globals_kw):
        kv = prefill + steps + 1
        if generate_on_device:
            gpu = make_synthetic_mixtral(config, "cuda", seed, full=True, kv_positions=kv, prefill=prefill,
                                         ln_weight_std=ln_weight_std, predictor_sigma=predictor_sigma)
            self.gpu_model, self.cpu_model = gpu, to_device(gpu, "cpu")
        else:
            cpu = make_synthetic_mixtral(config, "cpu", seed, full=True, kv_positions=kv, prefill=prefill,
                                         ln_weight_std=ln_weight_std, predictor_sigma=predictor_sigma)
            self.cpu_model, self.gpu_model = cpu, to_device(cpu, "cuda")
        if workers is None:
            workers = torch.cuda.get_device_properties(0).multi_processor_count
        self.g_cpu = make_globals(self.cpu_model, sm_count=workers, seq_len=prefill, **globals_kw)
        self.g_gpu = make_globals(self.gpu_model, sm_count=workers, seq_len=prefill, **globals_kw)
        self.g_gpu.pos_id = self.g_cpu.pos_id = prefill
        dag_kw = {"predict": predict}
        if start_after_op is None:
            nodes, end = make_dag(self.g_gpu, stop_after_op=stop_after_op, layer_limit=layer_limit, **dag_kw)
            self.schedule = Schedule(self.g_gpu, nodes, end)
            self.prefix = []
            self.linear = self.schedule.get_linear_instructions()
            queues = assign_to_sms(mode, schedule=self.schedule)
        else:
            self.prefix, self.linear = split_linear(make_dag, self.g_gpu, start_after_op, layer_limit, stop_after_op,
                                                    **dag_kw)
            assert mode in ("rr", "zz"), "a schedule suffix is assigned from its instruction list"
            queues = assign_to_sms(mode, instructions=self.linear, sm_count=workers)
        self.g_cpu.skip_attn_reduction = self.g_gpu.skip_attn_reduction
        tensorize_instructions(self.g_gpu, queues)
        self.pos = prefill

    def step(self, token: int, **kw):
        import mk_mixtral
        from megakernels_amd.mixtral.mk import interpret_with_mk

        for g, model in ((self.g_cpu, self.cpu_model), (self.g_gpu, self.gpu_model)):
            g.hidden_states.copy_(model.embed_tokens[token])
            g.barriers.zero_()
            g.logits.zero_()
            g.pos_id = self.pos
        if self.prefix:
            oracle.interpret_with_pyvm(self.g_cpu, self.prefix)
            copy_state(self.g_gpu, self.g_cpu)
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

    def agreement(self) -> dict:
        """(max bf16 ulps, bit-identical fraction) of the bf16 outputs of the
        step against the oracle: the last layer's normed hidden and SiLU rows
        of the selected experts, the residual, the new K/V rows, q, the
        attention output and the logits."""
        g, r = self.g_gpu, self.g_cpu
        pos = self.pos - 1
        idx = r.selected_expert_indices.long()
        out = {
            "hidden": bf16_agreement(g.hidden_states, r.hidden_states),
            "normed": bf16_agreement(g.router_normed_hidden, r.router_normed_hidden),
            "silu": bf16_agreement(g.expert_silu_out.cpu()[idx], r.expert_silu_out[idx]),
            "k_new": bf16_agreement(g.k_cache[:, 0, pos], r.k_cache[:, 0, pos]),
            "v_new": bf16_agreement(g.v_cache[:, 0, pos], r.v_cache[:, 0, pos]),
            "q": bf16_agreement(g.post_ln_rope_q, r.post_ln_rope_q),
            "attn_out": bf16_agreement(g.attn_out, r.attn_out),
        }
        if r.logits.any():
            out["logits"] = bf16_agreement(g.logits, r.logits)
        return out

    def barriers_equal(self) -> bool:
        return torch.equal(self.g_gpu.barriers.cpu(), self.g_cpu.barriers)

    def indices(self):
        return self.g_gpu.selected_expert_indices.cpu().tolist(), self.g_cpu.selected_expert_indices.tolist()
