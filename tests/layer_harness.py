"""One layer of a full-size model, stage by stage, on the GPU against the CPU
oracle run on that layer's weights alone.

The whole-model tests at the config shapes either slice the model to its
first two layers (oracle comparisons) or check properties that hold at any
size (the full 32- and 28-layer models): neither reads a weight or cache
byte of a deep layer and compares the value.  Here the kernel runs the
stages of layer ``layer`` (the last one, say) of the full tensors -- its
expert rows sit tens of GiB into ``expert_gate_weights``, its K/V rows
gigabytes into the caches -- while the oracle runs the same stages as layer
0 of a one-layer copy of that layer's weights and cache.

Each stage starts from the oracle's own state, as the reference's diff
harness does (megakernels/scripts/diff_test.py:139-162): the residual is
drawn, the stages before ``after`` run on the oracle, its state (with its
layer-0 barrier row as the kernel's row ``layer``, and the previous layer's
down-projection counter filled) is copied to the GPU, and the stages from
``after`` through ``through`` run on both.  So the stage under test sees
bit-identical inputs and its outputs can be held to the rounding-point bar.
"""

from __future__ import annotations

from dataclasses import replace
from types import SimpleNamespace

import torch

from megakernels_amd.scheduler import assign_to_sms, tensorize_instructions
from moe_harness import bf16_agreement, max_abs_rel


def slice_layer(model, layer: int, device="cpu"):
    """A one-layer copy of ``model`` (Mixtral or dense Llama synthetic
    model) holding layer ``layer``'s weights, norms and KV cache; the
    embeddings, LM head and RoPE tables are copied whole."""
    L = model.config.num_hidden_layers
    device = torch.device(device)

    def mv(t, cut=True):
        if t is None:
            return None
        if cut and t.dim() > 0 and t.shape[0] == L:
            t = t[layer:layer + 1]
        return t.to(device).contiguous()

    sp = model.stacked_params
    return SimpleNamespace(
        config=replace(model.config, num_hidden_layers=1),
        device=device,
        dtype=model.dtype,
        stacked_params=type(sp)(**{k: mv(v) for k, v in vars(sp).items()}),
        lm_head=SimpleNamespace(input_norm=SimpleNamespace(weight=mv(model.lm_head.input_norm.weight, False)),
                                lm_head=SimpleNamespace(weight=mv(model.lm_head.lm_head.weight, False))),
        embed_tokens=mv(model.embed_tokens, False),
        stacked_kv_cache=tuple(mv(t) for t in model.stacked_kv_cache),
        model=SimpleNamespace(rope_cos=mv(model.model.rope_cos, False), rope_sin=mv(model.model.rope_sin, False)),
        generator=None,
    )


def stage_instructions(dag_layer, globs, layer: int, after: str | None, through: str | None, **kw):
    """Instructions of layer ``layer`` after stage ``after`` (None: from the
    layer's start) through stage ``through`` (None: the whole layer), in the
    DAG's topological order."""
    nodes, _ = dag_layer(globs, layer, [], stop_after_op=through, **kw)
    full = [n.instruction for n in nodes]
    if after is None:
        return full
    pre = [n.instruction for n in dag_layer(globs, layer, [], stop_after_op=after, **kw)[0]]
    assert len(pre) < len(full) and full[:len(pre)] == pre, f"{after} is not a prefix of {through}"
    return full[len(pre):]


class LayerCase:
    def __init__(self, gpu_model, layer: int, pos: int, workers: int | None = None):
        self.dense = hasattr(gpu_model.stacked_params, "gate_proj")
        if self.dense:
            from megakernels_amd.latency.scheduler import expected_downproj_arrivals, make_dag_layer, make_globals
            from oracle import latency_vm as oracle

            self.dag_kw = {}
            self.state = ("hidden_states", "post_ln_rope_q", "attn_out", "attn_out_intermediates",
                          "attn_lse_intermediates", "silu_out", "logits")
        else:
            from megakernels_amd.mixtral.scheduler import expected_downproj_arrivals, make_dag_layer, make_globals
            from oracle import python_vm as oracle

            self.dag_kw = {"predict": True}
            self.state = ("hidden_states", "post_ln_rope_q", "attn_out", "attn_out_intermediates",
                          "attn_lse_intermediates", "expert_silu_out", "router_normed_hidden", "logits",
                          "selected_expert_indices", "selected_expert_scores", "predicted_expert_indices")
        self.oracle = oracle
        self.dag_layer = make_dag_layer
        if workers is None:
            workers = torch.cuda.get_device_properties(0).multi_processor_count
        self.workers = workers
        self.layer = layer
        self.pos = pos
        self.gpu_model = gpu_model
        self.cpu_model = slice_layer(gpu_model, layer, "cpu")
        self.g_gpu = make_globals(gpu_model, sm_count=workers, seq_len=pos)
        self.g_cpu = make_globals(self.cpu_model, sm_count=workers, seq_len=pos)
        self.g_gpu.pos_id = self.g_cpu.pos_id = pos
        self.prev_done = expected_downproj_arrivals(self.g_gpu)
        self.residual = None

    def run(self, after: str | None, through: str | None, residual: torch.Tensor):
        """The stages after ``after`` through ``through`` of the case's layer
        from the oracle's state, on both sides."""
        g, r, layer, pos = self.g_gpu, self.g_cpu, self.layer, self.pos
        gi = stage_instructions(self.dag_layer, g, layer, after, through, **self.dag_kw)
        ci = stage_instructions(self.dag_layer, r, 0, after, through, **self.dag_kw)
        assert [type(i) for i in gi] == [type(i) for i in ci]
        self.residual = residual.clone()
        r.hidden_states.copy_(residual)
        r.barriers.zero_()
        r.logits.zero_()
        if after is not None:
            self.oracle.interpret_with_pyvm(r, stage_instructions(self.dag_layer, r, 0, None, after, **self.dag_kw))
        for n in self.state:
            getattr(g, n).copy_(getattr(r, n))
        g.barriers.zero_()
        g.barriers[layer].copy_(r.barriers[0])
        if layer > 0:
            g.barriers[layer - 1, 5, 0] = self.prev_done
        g.k_cache[layer, :, pos].copy_(r.k_cache[0, :, pos])
        g.v_cache[layer, :, pos].copy_(r.v_cache[0, :, pos])
        self.expected_bars = g.barriers.cpu()
        tensorize_instructions(g, assign_to_sms("rr", instructions=gi, sm_count=self.workers))
        if self.dense:
            import mk_llama
            from megakernels_amd.latency.mk import interpret_with_mk

            interpret_with_mk(g, mk_llama.mk_llama, debug_sync=True)
        else:
            import mk_mixtral
            from megakernels_amd.mixtral.mk import interpret_with_mk

            interpret_with_mk(g, mk_mixtral.mk_mixtral, debug_sync=True)
        torch.cuda.synchronize()
        self.oracle.interpret_with_pyvm(r, ci)
        # the oracle's barrier row is the kernel's row `layer`; every other
        # row is what the launch started from
        self.expected_bars[layer] = r.barriers[0]

    def _pairs(self):
        g, r, layer, pos = self.g_gpu, self.g_cpu, self.layer, self.pos
        out = {
            "hidden": (g.hidden_states, r.hidden_states),
            "k_new": (g.k_cache[layer, 0, pos], r.k_cache[0, 0, pos]),
            "v_new": (g.v_cache[layer, 0, pos], r.v_cache[0, 0, pos]),
            "q": (g.post_ln_rope_q, r.post_ln_rope_q),
            "attn_out": (g.attn_out, r.attn_out),
        }
        if self.dense:
            out["silu"] = (g.silu_out, r.silu_out)
        else:
            idx = r.selected_expert_indices.long()
            out["normed"] = (g.router_normed_hidden, r.router_normed_hidden)
            out["silu"] = (g.expert_silu_out.cpu()[idx], r.expert_silu_out[idx])
        return out

    def errors(self) -> dict:
        return {k: max_abs_rel(a, b) for k, (a, b) in self._pairs().items() if b.float().abs().max() > 0}

    def agreement(self) -> dict:
        return {k: bf16_agreement(a, b) for k, (a, b) in self._pairs().items() if b.float().abs().max() > 0}

    def barriers_equal(self) -> bool:
        return torch.equal(self.g_gpu.barriers.cpu(), self.expected_bars)

    def predictor_margins(self):
        """The oracle's predictor logits of this layer, from the residual the
        stage started from (opcode 8 reads the pre-attention residual):
        (gap top-1 / top-2, gap top-2 / top-3)."""
        r = self.g_cpu
        normed = self.oracle.rms_norm(self.residual, r.ffn_ln_weights[0], r.rms_norm_eps)
        w = r.router_weights if r.predictor_weights is None else r.predictor_weights
        top = torch.sort(self.oracle.router_logits(w[0].contiguous(), normed), descending=True).values
        return float(top[0] - top[1]), float(top[1] - top[2])

    def router_margins(self):
        """The oracle's router-logit gaps of this layer (top-1 / top-2,
        top-2 / top-3) over the normed hidden its opcode 5 computed."""
        r = self.g_cpu
        top = torch.sort(self.oracle.router_logits(r.router_weights[0].contiguous(), r.router_normed_hidden),
                         descending=True).values
        return float(top[0] - top[1]), float(top[1] - top[2])
