"""Greedy batch-1 decode driver over the persistent kernel.

Counterpart of ``MK_Generator`` (``megakernels/generators.py:95-166``), for
the Mixtral VM and the dense Llama VM alike: a step embeds the input token
into ``hidden_states``, refills the barrier tensor, sets ``pos_id``, zeroes
the logits (the Mixtral LM head accumulates its column blocks into them),
launches the whole-model schedule once, and takes the argmax of the logits.
``generate`` runs steps back to back, feeding each output token to the next
step, as ``MK_Generator.generate`` does.

The argmax and the next step's embedding run inside the launch
(``argmax_out`` / ``next_embed_weights`` of the C ABI): the kernel's last
workgroup writes the token straight into ``output_tokens`` and copies its
embedding row into ``hidden_states``, where the reference runs
``torch.argmax`` and the embedding lookup between launches
(``megakernels/generators.py:121-145``).  It also zeroes the barriers and
the logits for the next launch (``reset_for_next_launch``), so a step after
the first enqueues the launch alone (``reset_next=False`` keeps the fills).
``device_argmax=False`` restores the torch calls and the fills.

Mixtral launches run with ``work_sharing`` on unless the caller says
otherwise: a workgroup that has finished its own opcode-5 rows takes the
last rows of the other workers of its group (one per XCD), which evens out
the XCDs' different streaming rates within each layer; every row is
computed the same way by whoever takes it, so the results are bit-identical
to a launch without it.

The schedule is built once (``make_dag`` over all layers plus the LM head)
and reused for every position; partial-attention instructions cover the
positions ``[0, pos_id]`` of their partition at run time.

The rest of the reference generator's surface is here too:
``generate_with_eos`` (chunks of steps with an end-of-sequence check on the
host after each chunk, ``megakernels/generators.py:21-58``), ``skip_mk`` and
``skip_rest`` (leave out the launch, or everything but the launch, to time
the other part, ``:100-103, 137-141``) and ``replace_with_noops`` (every
instruction becomes a NoOp: the launch costs only its fixed overhead,
``:118-119``).
"""

from __future__ import annotations

import time

import torch

from ..scheduler import Schedule, assign_to_sms, group_rows_by_xcd, tensorize_instructions
from .mk import MixtralMK_Interpreter
from .scheduler import make_dag, make_globals


class MK_Generator:
    def __init__(self, model, interpreter: MixtralMK_Interpreter, schedule: Schedule, barrier_fill_val: int = 0,
                 skip_mk: bool = False, skip_rest: bool = False, device_argmax: bool = True,
                 reset_next: bool = True, **launch_kwargs):
        self.model = model
        self.interpreter = interpreter
        self.schedule = schedule
        self.barrier_fill_val = barrier_fill_val
        # skip_mk: no launch (embedding, fills and argmax only); skip_rest:
        # the launch only, no embedding and no argmax (the input token is
        # passed through) -- megakernels/generators.py:100-103, 121-141
        self.skip_mk = skip_mk
        self.skip_rest = skip_rest
        self.device_argmax = device_argmax
        self.reset_next = reset_next and barrier_fill_val == 0
        self.launch_kwargs = launch_kwargs
        self.last_gpu_seconds = None
        self.fill()
        # the barriers and logits are zero (the last launch reset them)
        self._clean = False

    @classmethod
    def build(cls, model, prompt_len: int, mode: str = "rr", sm_count: int | None = None, dag_kwargs=None,
              globals_kwargs=None, xcd_rows=(), **launch_kwargs):
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
            launch_kwargs.setdefault("work_sharing", True)
        globs = globals_fn(model, seq_len=prompt_len, sm_count=sm_count, **(globals_kwargs or {}))
        globs.pos_id = prompt_len
        nodes, end = dag_fn(globs, **(dag_kwargs or {}))
        schedule = Schedule(globs, nodes, end)
        queues = assign_to_sms(mode, schedule=schedule)
        if xcd_rows:
            queues = group_rows_by_xcd(queues, xcd_rows)
        tensorize_instructions(globs, queues)
        return cls(model, interpreter, schedule, **launch_kwargs)

    def fill(self):
        self.schedule.globs.barriers.fill_(self.barrier_fill_val)

    def replace_with_noops(self):
        """Every queued instruction becomes a NoOp (opcode 0): a launch then
        costs only the kernel's fixed overhead (megakernels/generators.py:118-119)."""
        self.schedule.globs.instructions.zero_()

    def run(self, input_ids: torch.Tensor, pos_id: int) -> torch.Tensor:
        """One step from ``input_ids``; returns the output token (0-d)."""
        return self._step(input_ids, pos_id)

    def _step(self, input_ids, pos_id: int, out: torch.Tensor | None = None, embedded: bool = False,
              embed_next: bool = False) -> torch.Tensor:
        """One launch.  ``embedded``: the previous launch already wrote this
        step's input embedding into ``hidden_states``.  ``out``: a 0-d int64
        view the kernel writes the token into.  ``embed_next``: the launch
        also writes that token's embedding into ``hidden_states``."""
        globs = self.schedule.globs
        if not embedded and not self.skip_rest:
            globs.hidden_states.copy_(self.model.embed_tokens[input_ids.reshape(-1)[0]])
        if not self._clean:
            self.fill()
            globs.logits.zero_()
        globs.pos_id = pos_id
        if self.skip_mk or not self.device_argmax or self.skip_rest:
            self._clean = False
            if not self.skip_mk:
                self.interpreter.interpret(globs, **self.launch_kwargs)
            if self.skip_rest:
                return input_ids.reshape(-1)[0]
            return torch.argmax(globs.logits, dim=-1)
        if out is None:
            out = torch.empty((), dtype=torch.long, device=globs.logits.device)
        self._clean = False
        self.interpreter.interpret(globs, argmax_out=out,
                                   next_embed_weights=self.model.embed_tokens if embed_next else None,
                                   reset_for_next_launch=self.reset_next, **self.launch_kwargs)
        self._clean = self.reset_next
        return out

    def generate(self, output_tokens: torch.Tensor, prompt_len: int, ntok: int, ntok_already_generated: int = 1):
        """Fill ``output_tokens[:, ntok_already_generated : +ntok]`` greedily
        (``megakernels/generators.py:148-166``).  With the in-kernel argmax
        each launch writes its token into ``output_tokens`` and the embedding
        of that token for the next launch."""
        chain = (self.device_argmax and not (self.skip_mk or self.skip_rest) and output_tokens.dtype == torch.long
                 and output_tokens.shape[0] == 1 and output_tokens.is_contiguous())
        for i in range(ntok):
            input_pos = ntok_already_generated + i - 1
            input_ids = output_tokens[:, input_pos:input_pos + 1]
            pos_id = prompt_len + ntok_already_generated + i - 1
            if chain:
                self._step(input_ids, pos_id, out=output_tokens[0, input_pos + 1], embedded=i > 0,
                           embed_next=i + 1 < ntok)
            else:
                output_tokens[:, input_pos + 1] = self.run(input_ids, pos_id=pos_id)
        return output_tokens

    def generate_with_eos(self, output_tokens: torch.Tensor, prompt_len: int, ntok: int,
                          eos_token_check_interval: int, eos_token_ids: list[int]):
        """Greedy steps in chunks of ``eos_token_check_interval``, copying
        each chunk's tokens to the host and stopping at the first token in
        ``eos_token_ids``.  Returns (index in ``output_tokens`` of that
        token, tokens generated), or (ntok, ntok - 1) when none came
        (megakernels/generators.py:21-58; batch 1)."""
        if output_tokens.shape[0] != 1:
            raise ValueError("batch size must be 1")
        if eos_token_check_interval < 1:
            raise ValueError("eos_token_check_interval must be >= 1")
        eos = set(int(t) for t in eos_token_ids)
        for done in range(1, ntok, eos_token_check_interval):
            n = min(eos_token_check_interval, ntok - done)
            self.generate(output_tokens, prompt_len=prompt_len, ntok=n, ntok_already_generated=done)
            chunk = output_tokens[0, done:done + n].cpu().tolist()
            for j, tok in enumerate(chunk):
                if int(tok) in eos:
                    # the first token was given, not generated
                    return done + j, done + n - 1
        return ntok, ntok - 1

    def timed_generate(self, first_token: int, prompt_len: int, ntok: int, warmup: int = 2):
        """(tokens, seconds) of ``ntok`` greedy steps after ``warmup``
        untimed ones, bracketed by device synchronisations; the same span
        from HIP events on the launch stream is left in
        ``last_gpu_seconds``.  The warmup steps write positions that the
        timed steps then overwrite."""
        dev = self.schedule.globs.hidden_states.device
        tokens = torch.zeros(1, ntok + 1, dtype=torch.long, device=dev)
        tokens[0, 0] = first_token
        if warmup:
            self.generate(tokens.clone()[:, :warmup + 1], prompt_len, warmup)
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        start.record()
        self.generate(tokens, prompt_len, ntok)
        stop.record()
        torch.cuda.synchronize(dev)
        secs = time.perf_counter() - t0
        self.last_gpu_seconds = start.elapsed_time(stop) / 1e3
        return tokens, secs
