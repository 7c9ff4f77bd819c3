"""Repeated launches of one decode step give bit-identical results.

Every value a launch computes depends only on its inputs, whatever order
the workgroups run in, so a thousand launches of the same step must agree
bit for bit with the first.  The dense (Llama) VM at the config-3 shape
with one layer is the case that exposed a race: an opcode-5 instruction
that stages its own first up/gate items (one not preceded by an O
projection in its worker's queue) used to publish the staged count in
shared memory while its waves were still reading that word to decide
whether to stage, and a wave that saw the new value skipped the staging
and one workgroup barrier; from then on it ran one barrier ahead of the
others and read the workgroup's sum of squares before the other waves had
written theirs (the normed hidden state 1 ulp off in its 512 columns), or
computed its staged item from rows that were never loaded.  With three
staged items about 2.6 % of launches differed.  The sweep covers the
staging counts that exposed it and the default, and the Mixtral VM on a
two-layer slice (epic-kernel_amd/csrc/mk_mixtral.hip: stage_dense_upgate,
op_dense_upgate).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

FIELDS = ("MK_STAGE_ITEMS", "MK_CODE_PF")


@pytest.fixture(autouse=True)
def _clean_env(monkeypatch):
    for name in FIELDS:
        monkeypatch.delenv(name, raising=False)


def _reload():
    import mk_mixtral

    mk_mixtral.load_library().mk_mixtral_reload_overrides()


def _state(g, out, mixtral):
    s = {"token": out.clone(), "logits": g.logits.clone(), "hidden": g.hidden_states.clone(),
         "attn_out": g.attn_out.clone()}
    s["silu"] = (g.expert_silu_out if mixtral else g.silu_out).clone()
    if mixtral:
        s["sel"] = g.selected_expert_indices.clone()
    return s


def _repeat(gen, token, pos, launches, monkeypatch, variants, mixtral=False, **kw):
    g = gen.schedule.globs
    emb = gen.model.embed_tokens[token].clone()
    out = torch.full((), -1, dtype=torch.long, device="cuda")
    if mixtral:
        import mk_mixtral
        from megakernels_amd.mixtral.mk import interpret_with_mk

        fn = mk_mixtral.mk_mixtral
    else:
        import mk_llama
        from megakernels_amd.latency.mk import interpret_with_mk

        fn = mk_llama.mk_llama

    def launch():
        g.hidden_states.copy_(emb)
        g.barriers.zero_()
        g.logits.zero_()
        g.pos_id = pos
        interpret_with_mk(g, fn, argmax_out=out, debug_sync=True, **kw)
        return _state(g, out, mixtral)

    _reload()
    base = launch()
    torch.cuda.synchronize()
    assert bool(torch.isfinite(base["logits"].float()).all())
    for env in variants:
        for name, value in env.items():
            monkeypatch.setenv(name, value)
        _reload()
        print(f"[repeat {'mixtral' if mixtral else 'llama'}] {env or 'default'} x {launches}", flush=True)
        bad = []
        for i in range(launches):
            got = launch()
            diff = [k for k in base if not torch.equal(base[k], got[k])]
            if diff:
                bad.append((i, diff))
        for name in env:
            monkeypatch.delenv(name)
        _reload()
        assert not bad, f"{env}: {len(bad)} of {launches} launches differ from the first, e.g. {bad[:3]}"


def test_llama_one_layer_repeat_bit_identical(monkeypatch):
    from dataclasses import replace

    from megakernels_amd.latency.synthetic import C3, make_synthetic_llama
    from megakernels_amd.mixtral.generate import MK_Generator

    pos = 2048
    model = make_synthetic_llama(replace(C3, num_hidden_layers=1), "cuda", 61, kv_positions=pos + 4, prefill=pos)
    try:
        gen = MK_Generator.build(model, pos)
        _repeat(gen, 777, pos, 1500, monkeypatch,
                [{}, {"MK_STAGE_ITEMS": "3"}, {"MK_STAGE_ITEMS": "1"},
                 {"MK_STAGE_ITEMS": "3", "MK_CODE_PF": "0"}])
    finally:
        del model
        torch.cuda.empty_cache()


def test_mixtral_two_layer_repeat_bit_identical(monkeypatch):
    from megakernels_amd.mixtral.generate import MK_Generator
    from megakernels_amd.mixtral.synthetic import C4, make_synthetic_mixtral, with_layers

    pos = 4096
    model = make_synthetic_mixtral(with_layers(C4, 2), "cuda", 60, full=True, kv_positions=pos + 4, prefill=pos)
    try:
        gen = MK_Generator.build(model, pos)
        _repeat(gen, 1234, pos, 300, monkeypatch, [{}, {"MK_STAGE_ITEMS": "3"}], mixtral=True, work_sharing=True)
    finally:
        del model
        torch.cuda.empty_cache()
