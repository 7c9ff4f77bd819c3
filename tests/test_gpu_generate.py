"""Greedy decode through MK_Generator (megakernels_amd/mixtral/generate.py)
against the same loop over the CPU oracle PyVM (the reference's
PyVM_Generator, megakernels/generators.py:169-180): the generated token ids
must be the same, step by step, and so must the KV cache the steps append."""

import pytest
import torch

from megakernels_amd.mixtral.generate import MK_Generator
from megakernels_amd.mixtral.scheduler import make_dag, make_globals
from megakernels_amd.mixtral.synthetic import TINY, make_synthetic_mixtral, to_device
from megakernels_amd.scheduler import Schedule
from moe_harness import max_abs_rel
from oracle import python_vm as oracle

pytestmark = pytest.mark.gpu


def _oracle_generate(model, prompt_len, first, ntok, sm_count):
    g = make_globals(model, seq_len=prompt_len, sm_count=sm_count)
    g.pos_id = prompt_len
    nodes, end = make_dag(g)
    linear = Schedule(g, nodes, end).get_linear_instructions()
    toks = [first]
    for i in range(ntok):
        g.hidden_states.copy_(model.embed_tokens[toks[-1]])
        g.barriers.zero_()
        g.logits.zero_()
        g.pos_id = prompt_len + i
        oracle.interpret_with_pyvm(g, linear)
        toks.append(int(g.logits.float().argmax()))
    return toks, g


@pytest.mark.parametrize("prompt_len,device_argmax", [(40, True), (300, True), (40, False)])
def test_greedy_tokens_match_oracle(prompt_len, device_argmax):
    """device_argmax: the launch writes each token into ``tokens`` and the
    next input's embedding (the default); False: torch.argmax and the
    embedding lookup between launches, as the reference's generator."""
    ntok = 4
    cpu = make_synthetic_mixtral(TINY, "cpu", 21, full=True, kv_positions=prompt_len + ntok + 1,
                                 prefill=prompt_len, ln_weight_std=0.1)
    gpu = to_device(cpu, "cuda")
    gen = MK_Generator.build(gpu, prompt_len, device_argmax=device_argmax, debug_sync=True)
    W = gen.schedule.globs.sm_count()
    tokens = torch.zeros(1, ntok + 1, dtype=torch.long, device="cuda")
    tokens[0, 0] = 7
    gen.generate(tokens, prompt_len, ntok)
    ref, g_ref = _oracle_generate(cpu, prompt_len, 7, ntok, W)
    print(f"[generate] gpu {tokens[0].tolist()} oracle {ref}", flush=True)
    assert tokens[0].tolist() == ref
    for p in range(prompt_len, prompt_len + ntok):
        assert max_abs_rel(gpu.stacked_kv_cache[0][:, 0, p], g_ref.k_cache[:, 0, p]) <= 2e-2
        assert max_abs_rel(gpu.stacked_kv_cache[1][:, 0, p], g_ref.v_cache[:, 0, p]) <= 2e-2


def test_timed_generate_runs_without_host_syncs():
    cpu = make_synthetic_mixtral(TINY, "cpu", 22, full=True, kv_positions=64, prefill=32)
    gen = MK_Generator.build(to_device(cpu, "cuda"), 32)
    tokens, secs = gen.timed_generate(3, 32, 8, warmup=2)
    assert secs > 0 and tokens.shape == (1, 9) and int(tokens.min()) >= 0
    import mk_mixtral

    mk_mixtral.raise_if_failed("cuda")


def test_two_generators_on_two_streams():
    """Two decoders with their own weights, caches and barrier tensors,
    stepped alternately on two streams with no host synchronisation between
    the steps.  Launches on one device run one at a time (the library makes
    a launch on a new stream wait for the previous launch's stream), so both
    token streams equal the oracle's."""
    prompt_len, ntok = 40, 4
    cpus = [make_synthetic_mixtral(TINY, "cpu", seed, full=True, kv_positions=prompt_len + ntok + 1,
                                   prefill=prompt_len, ln_weight_std=0.1) for seed in (31, 32)]
    gens = [MK_Generator.build(to_device(c, "cuda"), prompt_len) for c in cpus]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    toks = [torch.zeros(1, ntok + 1, dtype=torch.long, device="cuda") for _ in gens]
    for t, first in zip(toks, (7, 9)):
        t[0, 0] = first
    torch.cuda.synchronize()
    for i in range(ntok):
        for gen, st, t in zip(gens, streams, toks):
            with torch.cuda.stream(st):
                gen.generate(t, prompt_len, 1, ntok_already_generated=i + 1)
    torch.cuda.synchronize()
    import mk_mixtral

    mk_mixtral.raise_if_failed("cuda")
    W = gens[0].schedule.globs.sm_count()
    for cpu, t, first in zip(cpus, toks, (7, 9)):
        ref, _ = _oracle_generate(cpu, prompt_len, first, ntok, W)
        print(f"[two streams] gpu {t[0].tolist()} oracle {ref}", flush=True)
        assert t[0].tolist() == ref
