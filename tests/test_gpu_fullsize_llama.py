"""Full-size properties of Llama-3.2-3B-shaped decode on the dense VM
28 layers, vocab 128256, the KV cache pre-filled to
2048 positions.  The two-layer slice at the same shape is checked against
the oracle in test_gpu_configs.py; here, what holds at any size:

* the token the launch writes equals torch.argmax of the logits it left;
* the barrier tensor equals its closed forms (lat/python_vm.py's arrivals):
  per layer every QKV head counter at head_dim / qkv_block_size, every query
  head's partial counter at the partition count, Hq reduced heads,
  H / o_proj_block_size O-proj blocks, F / up_gate_proj_block_size up/gate
  blocks and (F / matvec_reduction_size) (H / down_proj_block_size)
  down-projection chunks, zero elsewhere;
* a relaunch from the same input is bit-identical (token, logits, residual):
  with the default full-row down projection every residual row has one
  writer, which adds in python_vm's order; so is a launch with prefetch off
  (``late_loads``: no load before its wait, nothing staged in LDS).
"""

import pytest
import torch

from megakernels_amd.latency.synthetic import C3, make_synthetic_llama
from megakernels_amd.mixtral.generate import MK_Generator
from moe_harness import max_abs_rel

pytestmark = pytest.mark.gpu

PREFILL = 2048


@pytest.fixture(scope="module")
def model():
    m = make_synthetic_llama(C3, "cuda", 51, kv_positions=PREFILL + 4, prefill=PREFILL)
    torch.cuda.synchronize()
    yield m
    del m
    torch.cuda.empty_cache()


def _launch(gen, token: int, pos: int, **kw):
    import mk_llama
    from megakernels_amd.latency.mk import interpret_with_mk

    g = gen.schedule.globs
    g.hidden_states.copy_(gen.model.embed_tokens[token])
    g.barriers.zero_()
    g.logits.zero_()
    g.pos_id = pos
    out = torch.full((), -1, dtype=torch.long, device="cuda")
    interpret_with_mk(g, mk_llama.mk_llama, argmax_out=out, debug_sync=True, **kw)
    torch.cuda.synchronize()
    return out


def test_fullsize_dense_decode_properties(model):
    gen = MK_Generator.build(model, PREFILL)
    g = gen.schedule.globs
    linear = gen.schedule.get_linear_instructions()
    nparts = max(i.num_partials for i in linear if i.opcode() == 2)
    tok = _launch(gen, 777, PREFILL)
    logits = g.logits.cpu()
    assert bool(torch.isfinite(logits.float()).all()) and bool(logits.float().abs().max() > 0)
    assert int(tok) == int(torch.argmax(logits)), "in-launch argmax differs from torch.argmax"

    L, Hq, Hkv = g.num_hidden_layers, g.num_attention_heads, g.num_kv_heads
    bar = torch.zeros_like(g.barriers, device="cpu")
    bar[:, 0, :Hq + 2 * Hkv] = g.head_dim // g.qkv_block_size
    if not g.skip_attn_reduction:
        bar[:, 1, :Hq] = nparts
    bar[:, 2, 0] = Hq
    bar[:, 3, 0] = g.hidden_size // g.o_proj_block_size
    bar[:, 4, 0] = g.intermediate_size // g.up_gate_proj_block_size
    bar[:, 5, 0] = (g.intermediate_size // g.matvec_reduction_size) * (g.hidden_size // g.down_proj_block_size)
    assert torch.equal(g.barriers.cpu(), bar), "barrier tensor differs from its closed forms"

    assert g.matvec_reduction_size == g.intermediate_size
    hidden = g.hidden_states.cpu()
    tok2 = _launch(gen, 777, PREFILL)
    print(f"[fullsize c3] tokens {int(tok)} / {int(tok2)}, relaunch logits max-abs-rel "
          f"{max_abs_rel(g.logits, logits):.1e}", flush=True)
    assert int(tok2) == int(tok)
    assert torch.equal(g.logits.cpu(), logits), "relaunch changed the logits"
    assert torch.equal(g.hidden_states.cpu(), hidden), "relaunch changed the residual"
    tok3 = _launch(gen, 777, PREFILL, late_loads=True)
    assert int(tok3) == int(tok)
    assert torch.equal(g.logits.cpu(), logits), "prefetch off changed the logits"
    assert torch.equal(g.hidden_states.cpu(), hidden), "prefetch off changed the residual"


LAST_LAYER_STAGES = {
    (None, "qkv"): ("k_new", "v_new", "q"),
    ("qkv", "reduction"): ("attn_out",),
    ("reduction", "oproj"): ("hidden",),
    ("oproj", "upgate"): ("silu",),
    ("upgate", "downproj"): ("hidden",),
}


@pytest.mark.parametrize("stage", list(LAST_LAYER_STAGES), ids=lambda s: f"{s[0] or 'start'}-{s[1]}")
def test_last_layer_stage_against_oracle(model, stage):
    """Layer 27 of the 28-layer 3B-shaped model against the dense oracle on a
    one-layer copy of its weights and cache, stage by stage from the
    oracle's state: outputs at least 99 % bit-identical, the barrier row
    equal."""
    from layer_harness import LayerCase
    from moe_harness import MIN_EXACT

    last = model.config.num_hidden_layers - 1
    case = LayerCase(model, last, PREFILL)
    g = torch.Generator().manual_seed(77)
    for _ in range(2):
        x = torch.randn(case.g_cpu.hidden_size, generator=g).to(torch.bfloat16)
        case.run(*stage, x)
        err, agr = case.errors(), case.agreement()
        tag = f"layer {last} {stage}"
        print(f"[{tag}] " + " ".join(f"{k} {v:.1e}" for k, v in err.items()), flush=True)
        print(f"[{tag}] ulp/exact " + " ".join(f"{k} {u}/{e:.4f}" for k, (u, e) in agr.items()), flush=True)
        for k, v in err.items():
            assert v <= 2e-2, f"{tag} {k}: max-abs-rel {v:.3e}"
        for k in LAST_LAYER_STAGES[stage]:
            assert agr[k][1] >= MIN_EXACT, f"{tag} {k}: {agr[k][1]:.4f} bit-identical"
        assert case.barriers_equal(), f"{tag}: barrier tensor differs"
