"""Launch-time tuning fields leave every result unchanged.

The host fills these fields of each launch from compile-time defaults, and
environment variables override them for measurements
(epic-kernel_amd/csrc/mk_mixtral.hip: ``tuning_value``, ``spread_layout``,
``stage_limit`` and the two launch paths):

* ``MK_SPIN_SLEEP``: the longest back-off between two polls of a counter;
* ``MK_TAIL``: the opcode-5 items of an instruction that other workers of
  its group may take (work sharing);
* ``MK_EARLY``: whether opcode 6 loads each wave's two first items into
  registers before the wait or after it;
* ``MK_PF``: the opcode-6 cache-warming rounds;
* ``MK_SPREAD``: which opcodes' counters are spread over per-XCD parts;
* ``MK_STAGE_ITEMS``: the predicted or next up/gate items staged in LDS;
* ``MK_CODE_PF``: whether every instruction start reads a slice of the
  kernel's machine code into L2 (0: off).

They decide when loads are issued, how long a poll sleeps, which workgroup
computes an item and where a counter's arrivals land, never the order of
any arithmetic, so a launch under any value is bit-identical to the default
launch: token (argmax inside the launch), logits, residual, the appended K
and V rows, the selected experts, and the barrier tensor.  Each variant
runs on a two-layer slice at the exact config-4 (Mixtral-8x7B, 4096 cached
positions) or config-3 (Llama-3.2-3B, 2048 cached) shape, so every path
runs at its real trip counts.  The library reads the environment once per
process; the test has it read again (``mk_mixtral_reload_overrides``) after
each change.
"""

import pytest
import torch

from megakernels_amd.latency.synthetic import C3, make_synthetic_llama
from megakernels_amd.mixtral.generate import MK_Generator
from megakernels_amd.mixtral.synthetic import C4, make_synthetic_mixtral, with_layers

pytestmark = pytest.mark.gpu

FIELDS = ("MK_SPIN_SLEEP", "MK_TAIL", "MK_EARLY", "MK_PF", "MK_SPREAD", "MK_STAGE_ITEMS")

#: (variable, value): both ends of each clamp range that the kernel accepts
#: (MK_TAIL 4096: every item of an instruction goes through the cursor, no
#: own-item loop and no staged rows used), a middle value, spreading off and
#: on for opcode 5 alone, staging off and partial, and a malformed value,
#: which is ignored
VARIANTS = [
    ("MK_SPIN_SLEEP", "1"), ("MK_SPIN_SLEEP", "64"),
    ("MK_TAIL", "1"), ("MK_TAIL", "64"), ("MK_TAIL", "4096"),
    ("MK_EARLY", "0"), ("MK_EARLY", "1"),
    ("MK_PF", "0"), ("MK_PF", "2"), ("MK_PF", "4"),
    ("MK_SPREAD", "0"), ("MK_SPREAD", "0x20"),
    ("MK_STAGE_ITEMS", "0"), ("MK_STAGE_ITEMS", "3"),
    ("MK_CODE_PF", "0"),
    ("MK_TAIL", "8x"),
]

MIXTRAL_POS = 4096
LLAMA_POS = 2048


@pytest.fixture(autouse=True)
def _clean_env(monkeypatch):
    for name in FIELDS:
        monkeypatch.delenv(name, raising=False)


def _launch(gen, lib, token: int, pos: int, **kw):
    g = gen.schedule.globs
    g.hidden_states.copy_(gen.model.embed_tokens[token])
    g.barriers.zero_()
    g.logits.zero_()
    g.pos_id = pos
    out = torch.full((), -1, dtype=torch.long, device="cuda")
    if lib == "mixtral":
        import mk_mixtral
        from megakernels_amd.mixtral.mk import interpret_with_mk

        interpret_with_mk(g, mk_mixtral.mk_mixtral, argmax_out=out, debug_sync=True, **kw)
    else:
        import mk_llama
        from megakernels_amd.latency.mk import interpret_with_mk

        interpret_with_mk(g, mk_llama.mk_llama, argmax_out=out, debug_sync=True, **kw)
    torch.cuda.synchronize()
    state = {"token": out.cpu(), "logits": g.logits.cpu(), "hidden": g.hidden_states.cpu(),
             "k": g.k_cache[:, 0, pos].cpu(), "v": g.v_cache[:, 0, pos].cpu(), "barriers": g.barriers.cpu()}
    if lib == "mixtral":
        state["sel"] = g.selected_expert_indices.cpu()
    return state


def _reload():
    import mk_mixtral

    mk_mixtral.load_library().mk_mixtral_reload_overrides()


def _sweep(gen, lib, token, pos, monkeypatch, **kw):
    _reload()
    base = _launch(gen, lib, token, pos, **kw)
    assert bool(torch.isfinite(base["logits"].float()).all()) and bool(base["logits"].float().abs().max() > 0)
    assert int(base["token"]) == int(torch.argmax(base["logits"]))
    for name, value in VARIANTS:
        print(f"[launch fields {lib}] {name}={value}", flush=True)
        monkeypatch.setenv(name, value)
        _reload()
        got = _launch(gen, lib, token, pos, **kw)
        monkeypatch.delenv(name)
        _reload()
        for k in base:
            assert torch.equal(base[k], got[k]), f"{name}={value} changed {k}"


def test_mixtral_launch_fields_bit_identical(monkeypatch):
    model = make_synthetic_mixtral(with_layers(C4, 2), "cuda", 60, full=True, kv_positions=MIXTRAL_POS + 4,
                                   prefill=MIXTRAL_POS)
    try:
        gen = MK_Generator.build(model, MIXTRAL_POS)
        # work sharing on, as the decode driver launches it: the tail field
        # only acts there
        _sweep(gen, "mixtral", 1234, MIXTRAL_POS, monkeypatch, work_sharing=True)
    finally:
        del model
        torch.cuda.empty_cache()


def test_llama_launch_fields_bit_identical(monkeypatch):
    from dataclasses import replace

    model = make_synthetic_llama(replace(C3, num_hidden_layers=2), "cuda", 61, kv_positions=LLAMA_POS + 4,
                                 prefill=LLAMA_POS)
    try:
        gen = MK_Generator.build(model, LLAMA_POS)
        _sweep(gen, "llama", 777, LLAMA_POS, monkeypatch)
    finally:
        del model
        torch.cuda.empty_cache()
