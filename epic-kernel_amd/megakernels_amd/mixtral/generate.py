"""Greedy batch-1 decode driver over the persistent kernel.

Counterpart of ``MK_Generator`` (``megakernels/generators.py:95-166``), for
the Mixtral VM and the dense Llama VM alike: a step embeds the input token into ``hidden_states``, refills the barrier
tensor, sets ``pos_id``, zeroes the logits (the LM head accumulates its
column blocks into them), launches the whole-model schedule once, and takes
the argmax of the logits.  ``generate`` runs steps back to back, feeding each
output token to the next step, as ``MK_Generator.generate`` does.

The schedule is built once (``make_dag`` over all layers plus the LM head)
and reused for every position; partial-attention instructions cover the
positions ``[0, pos_id]`` of their partition at run time.
"""

from __future__ import annotations

import time

import torch

from ..scheduler import Schedule, assign_to_sms, tensorize_instructions
from .mk import MixtralMK_Interpreter
from .scheduler import make_dag, make_globals


class MK_Generator:
    def __init__(self, model, interpreter: MixtralMK_Interpreter, schedule: Schedule, barrier_fill_val: int = 0,
                 **launch_kwargs):
        self.model = model
        self.interpreter = interpreter
        self.schedule = schedule
        self.barrier_fill_val = barrier_fill_val
        self.launch_kwargs = launch_kwargs
        self.fill()

    @classmethod
    def build(cls, model, prompt_len: int, mode: str = "rr", sm_count: int | None = None, dag_kwargs=None,
              globals_kwargs=None, **launch_kwargs):
        """Globals for ``model`` with the KV cache filled up to ``prompt_len``
        positions, the whole-model schedule assigned with ``mode``, and a
        generator over it.  The model type picks the VM: a model with
        ``stacked_params.expert_gate`` is Mixtral, one with
        ``stacked_params.gate_proj`` the dense Llama VM
        (``megakernels/dispatch.py`` maps model types the same way).
        ``dag_kwargs`` go to the VM's ``make_dag`` (e.g. ``predict=False``),
        ``globals_kwargs`` to its ``make_globals`` (block sizes, partition
        policy)."""
        if hasattr(model.stacked_params, "gate_proj"):
            from ..latency.mk import LatencyMK_Interpreter
            from ..latency.scheduler import make_dag as dag_fn
            from ..latency.scheduler import make_globals as globals_fn

            interpreter = LatencyMK_Interpreter()
        else:
            dag_fn, globals_fn, interpreter = make_dag, make_globals, MixtralMK_Interpreter()
        globs = globals_fn(model, seq_len=prompt_len, sm_count=sm_count, **(globals_kwargs or {}))
        globs.pos_id = prompt_len
        nodes, end = dag_fn(globs, **(dag_kwargs or {}))
        schedule = Schedule(globs, nodes, end)
        tensorize_instructions(globs, assign_to_sms(mode, schedule=schedule))
        return cls(model, interpreter, schedule, **launch_kwargs)

    def fill(self):
        self.schedule.globs.barriers.fill_(self.barrier_fill_val)

    def run(self, input_ids: torch.Tensor, pos_id: int) -> torch.Tensor:
        globs = self.schedule.globs
        globs.hidden_states.copy_(self.model.embed_tokens[input_ids.reshape(-1)[0]])
        self.fill()
        globs.pos_id = pos_id
        globs.logits.zero_()
        self.interpreter.interpret(globs, **self.launch_kwargs)
        return torch.argmax(globs.logits, dim=-1)

    def generate(self, output_tokens: torch.Tensor, prompt_len: int, ntok: int, ntok_already_generated: int = 1):
        """Fill ``output_tokens[:, ntok_already_generated : +ntok]`` greedily
        (``megakernels/generators.py:148-166``)."""
        for i in range(ntok):
            input_pos = ntok_already_generated + i - 1
            input_ids = output_tokens[:, input_pos:input_pos + 1]
            pos_id = prompt_len + ntok_already_generated + i - 1
            output_tokens[:, input_pos + 1] = self.run(input_ids, pos_id=pos_id)
        return output_tokens

    def timed_generate(self, first_token: int, prompt_len: int, ntok: int, warmup: int = 2):
        """(tokens, seconds) of ``ntok`` greedy steps after ``warmup``
        untimed ones, bracketed by device synchronisations.  The warmup steps
        write positions that the timed steps then overwrite."""
        dev = self.schedule.globs.hidden_states.device
        tokens = torch.zeros(1, ntok + 1, dtype=torch.long, device=dev)
        tokens[0, 0] = first_token
        if warmup:
            self.generate(tokens.clone()[:, :warmup + 1], prompt_len, warmup)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        self.generate(tokens, prompt_len, ntok)
        torch.cuda.synchronize(dev)
        return tokens, time.perf_counter() - t0
