"""The decode driver's host logic on the CPU (no launches): the generator
surface of megakernels/generators.py:21-166 -- generate_with_eos, skip_mk,
skip_rest, replace_with_noops -- driven by a scripted stand-in for the
kernel that writes the logits a launch would leave, and the schedule split
of the stage harness (megakernels/scripts/diff_test.py:139-153)."""

import pytest
import torch

from full_harness import split_linear
from megakernels_amd.latency.scheduler import make_dag as llama_dag
from megakernels_amd.latency.scheduler import make_globals as llama_globals
from megakernels_amd.latency.synthetic import LLAMA_TINY, make_synthetic_llama
from megakernels_amd.mixtral.generate import MK_Generator
from megakernels_amd.mixtral.scheduler import make_dag, make_globals
from megakernels_amd.mixtral.synthetic import TINY, make_synthetic_mixtral
from megakernels_amd.scheduler import Schedule, assign_to_sms, tensorize_instructions


class ScriptedKernel:
    """Leaves logits whose argmax is the next token of ``script`` (one per
    launch) and records the positions it was launched at."""

    def __init__(self, script):
        self.script = list(script)
        self.positions = []

    def interpret(self, globs, **kw):
        globs.logits.zero_()
        globs.logits[self.script[len(self.positions)]] = 1.0
        self.positions.append(int(globs.pos_id))


def _generator(script, prompt_len=8, **kw):
    model = make_synthetic_mixtral(TINY, "cpu", 3, full=True, kv_positions=64, prefill=prompt_len)
    g = make_globals(model, seq_len=prompt_len, sm_count=8)
    nodes, end = make_dag(g)
    sched = Schedule(g, nodes, end)
    tensorize_instructions(g, assign_to_sms("rr", schedule=sched))
    kernel = ScriptedKernel(script)
    return MK_Generator(model, kernel, sched, device_argmax=False, **kw), kernel, model


def test_generate_feeds_each_token_to_the_next_step():
    gen, kernel, model = _generator([5, 6, 7])
    toks = torch.zeros(1, 4, dtype=torch.long)
    toks[0, 0] = 2
    gen.generate(toks, prompt_len=8, ntok=3)
    assert toks[0].tolist() == [2, 5, 6, 7]
    assert kernel.positions == [8, 9, 10]
    # the last step's input was token 6's embedding
    assert torch.equal(gen.schedule.globs.hidden_states, model.embed_tokens[6])


@pytest.mark.parametrize("interval", [1, 2, 3, 5])
def test_generate_with_eos_stops_at_first_eos(interval):
    """Reference semantics: (index of the first EOS in output_tokens, tokens
    generated in the chunks run); the chunk holding the EOS is finished."""
    script = [5, 6, 99, 7, 8, 9, 10, 11]
    gen, kernel, _ = _generator(script)
    toks = torch.zeros(1, 9, dtype=torch.long)
    toks[0, 0] = 2
    first, total = gen.generate_with_eos(toks, prompt_len=8, ntok=8, eos_token_check_interval=interval,
                                        eos_token_ids=[99, 100])
    assert first == 3  # output index of token 99
    chunks_run = -(-3 // interval)
    assert total == min(chunks_run * interval, 7)
    assert len(kernel.positions) == total
    assert toks[0, :4].tolist() == [2, 5, 6, 99]


def test_generate_with_eos_without_eos():
    gen, kernel, _ = _generator([5, 6, 7, 8, 9])
    toks = torch.zeros(1, 6, dtype=torch.long)
    assert gen.generate_with_eos(toks, 8, 5, 2, [99]) == (5, 4)
    assert len(kernel.positions) == 4  # steps 1..4 (the first token is given)


def test_skip_mk_launches_nothing():
    gen, kernel, _ = _generator([5], skip_mk=True)
    toks = torch.zeros(1, 3, dtype=torch.long)
    gen.generate(toks, 8, 2)
    assert kernel.positions == []
    assert toks[0].tolist() == [0, 0, 0]  # argmax of zeroed logits


def test_skip_rest_launches_only():
    gen, kernel, model = _generator([5, 6], skip_rest=True)
    gen.schedule.globs.hidden_states.fill_(3.0)
    toks = torch.zeros(1, 3, dtype=torch.long)
    toks[0, 0] = 4
    gen.generate(toks, 8, 2)
    assert kernel.positions == [8, 9]
    assert toks[0].tolist() == [4, 4, 4]  # the input passed through
    assert bool((gen.schedule.globs.hidden_states == 3.0).all())  # no embedding


def test_replace_with_noops():
    gen, _, _ = _generator([5])
    assert bool(gen.schedule.globs.instructions.any())
    gen.replace_with_noops()
    assert not bool(gen.schedule.globs.instructions.any())


@pytest.mark.parametrize("start", ["qkv", "partial", "reduction", "oproj", "rms_router_upgate"])
def test_split_linear_mixtral(start):
    model = make_synthetic_mixtral(TINY, "cpu", 1, full=True, kv_positions=400, prefill=300)
    g = make_globals(model, seq_len=300, sm_count=16)
    prefix, suffix = split_linear(make_dag, g, start, None)
    nodes, end = make_dag(g)
    full = Schedule(g, nodes, end).get_linear_instructions()
    assert prefix + suffix == full and prefix and suffix
    last = {"qkv": 8, "partial": 2, "reduction": 3, "oproj": 4, "rms_router_upgate": 5}[start]
    assert prefix[-1].opcode() == last and all(i.layer_idx == 0 for i in prefix)


@pytest.mark.parametrize("start", ["qkv", "reduction", "oproj", "upgate"])
def test_split_linear_llama(start):
    model = make_synthetic_llama(LLAMA_TINY, "cpu", 1, kv_positions=400, prefill=300)
    g = llama_globals(model, seq_len=300, sm_count=16)
    prefix, suffix = split_linear(llama_dag, g, start, None)
    nodes, end = llama_dag(g)
    assert prefix + suffix == Schedule(g, nodes, end).get_linear_instructions()


def test_split_linear_rejects_a_non_prefix():
    model = make_synthetic_mixtral(TINY, "cpu", 1, full=True, kv_positions=40, prefill=20)
    g = make_globals(model, seq_len=20, sm_count=16)

    def rotated(gl, stop_after_op=None, layer_limit=None):
        # the whole schedule in another order than its stage prefix
        nodes, end = make_dag(gl, stop_after_op=stop_after_op, layer_limit=layer_limit)
        return (nodes[1:] + nodes[:1] if stop_after_op is None else nodes), end

    with pytest.raises(AssertionError, match="prefix"):
        split_linear(rotated, g, "oproj", None)
