"""Full-size properties of Mixtral-8x7B-shaped decode (BASELINE configs 4
and 5): all 32 layers, vocab 32000, 94 GB of weights resident, the KV cache
pre-filled to 16384 positions.  The oracle cannot hold this model on the
host, so these check what holds at any size (the two-layer slices at the
same shapes are checked against the oracle in test_gpu_configs.py):

* the token the launch writes (argmax inside the launch) equals
  torch.argmax of the logits the same launch left, on the CPU;
* the barrier tensor equals its closed forms (mkm/python_vm.py:38-54 and the
  arrivals of each solver): per layer, every QKV head counter at
  head_dim / qkv_block_size, every query head's partial counter at the
  partition count, Hq reduced heads, H / o_proj_block_size O-proj blocks,
  F / expert_proj_block_size up/gate blocks, 2 H / down_proj_block_size
  down blocks and one prediction, and zero elsewhere;
* a relaunch from the same input is bit-identical (token, logits, residual,
  the appended K/V rows): the Mixtral path adds in a fixed order; so is a
  launch with prefetch off (``late_loads``: no load before its wait, no
  predicted expert rows staged in LDS), which reads the same values later,
  and one with work sharing (idle workers take other workers' last
  opcode-5 rows, each computed the same way);
* the logits are finite and not all zero.

Config 4 decodes at position 4096 and config 5 at 16384 (predictor weights =
router + N(0, 0.007)), from one model.
"""

import pytest
import torch

from megakernels_amd.mixtral.generate import MK_Generator
from megakernels_amd.mixtral.synthetic import C4, make_synthetic_mixtral

pytestmark = pytest.mark.gpu

PREFILL_C5 = 16384


@pytest.fixture(scope="module")
def model():
    m = make_synthetic_mixtral(C4, "cuda", 50, full=True, kv_positions=PREFILL_C5 + 4, prefill=PREFILL_C5,
                               predictor_sigma=0.007)
    torch.cuda.synchronize()
    print(f"[fullsize] {torch.cuda.memory_allocated() / 1e9:.1f} GB allocated", flush=True)
    yield m
    del m
    torch.cuda.empty_cache()


def _launch(gen, token: int, pos: int, **kw):
    import mk_mixtral
    from megakernels_amd.mixtral.mk import interpret_with_mk

    g = gen.schedule.globs
    g.hidden_states.copy_(gen.model.embed_tokens[token])
    g.barriers.zero_()
    g.logits.zero_()
    g.pos_id = pos
    out = torch.full((), -1, dtype=torch.long, device="cuda")
    interpret_with_mk(g, mk_mixtral.mk_mixtral, argmax_out=out, debug_sync=True, **kw)
    torch.cuda.synchronize()
    return out


def expected_barriers(g, nparts: int) -> torch.Tensor:
    L, Hq, Hkv = g.num_hidden_layers, g.num_attention_heads, g.num_kv_heads
    bar = torch.zeros_like(g.barriers, device="cpu")
    bar[:, 0, :Hq + 2 * Hkv] = g.head_dim // g.qkv_block_size
    if not g.skip_attn_reduction:
        bar[:, 1, :Hq] = nparts
    bar[:, 2, 0] = Hq
    bar[:, 3, 0] = g.hidden_size // g.o_proj_block_size
    bar[:, 4, 0] = g.intermediate_size // g.expert_proj_block_size
    bar[:, 5, 0] = g.num_experts_per_tok * (g.hidden_size // g.down_proj_block_size)
    bar[:, 7, 0] = 1
    return bar


@pytest.mark.parametrize("pos", [4096, PREFILL_C5], ids=["c4", "c5"])
def test_fullsize_decode_properties(model, pos):
    gen = MK_Generator.build(model, pos)
    g = gen.schedule.globs
    nparts = max(i.num_partials for i in gen.schedule.get_linear_instructions() if i.opcode() == 2)
    print(f"[fullsize pos {pos}] {len(gen.schedule.dag_nodes)} instructions, {nparts} partitions", flush=True)
    tok = _launch(gen, 1234, pos)
    logits = g.logits.cpu()
    assert bool(torch.isfinite(logits.float()).all()) and bool(logits.float().abs().max() > 0)
    ref_tok = int(torch.argmax(logits))
    assert int(tok) == ref_tok, f"in-launch argmax {int(tok)} != torch.argmax {ref_tok}"
    assert torch.equal(g.barriers.cpu(), expected_barriers(g, nparts)), "barrier tensor differs from its closed forms"

    first = {"logits": logits.clone(), "hidden": g.hidden_states.cpu(), "k": g.k_cache[:, 0, pos].cpu(),
             "v": g.v_cache[:, 0, pos].cpu(), "sel": g.selected_expert_indices.cpu(),
             "pred": g.predicted_expert_indices.cpu()}
    tok2 = _launch(gen, 1234, pos)
    assert int(tok2) == int(tok)
    again = {"logits": g.logits.cpu(), "hidden": g.hidden_states.cpu(), "k": g.k_cache[:, 0, pos].cpu(),
             "v": g.v_cache[:, 0, pos].cpu(), "sel": g.selected_expert_indices.cpu(),
             "pred": g.predicted_expert_indices.cpu()}
    for k in first:
        assert torch.equal(first[k], again[k]), f"relaunch changed {k}"
    tok3 = _launch(gen, 1234, pos, late_loads=True)
    assert int(tok3) == int(tok)
    late = {"logits": g.logits.cpu(), "hidden": g.hidden_states.cpu(), "k": g.k_cache[:, 0, pos].cpu(),
            "v": g.v_cache[:, 0, pos].cpu(), "sel": g.selected_expert_indices.cpu(),
            "pred": g.predicted_expert_indices.cpu()}
    for k in first:
        assert torch.equal(first[k], late[k]), f"prefetch off changed {k}"
    # idle workers taking other workers' opcode-5 rows compute each row the
    # same way: bit-identical again
    tok4 = _launch(gen, 1234, pos, work_sharing=True)
    assert int(tok4) == int(tok)
    assert torch.equal(g.barriers.cpu(), expected_barriers(g, nparts)), "work sharing: barrier tensor differs"
    shared = {"logits": g.logits.cpu(), "hidden": g.hidden_states.cpu(), "k": g.k_cache[:, 0, pos].cpu(),
              "v": g.v_cache[:, 0, pos].cpu(), "sel": g.selected_expert_indices.cpu(),
              "pred": g.predicted_expert_indices.cpu()}
    for k in first:
        assert torch.equal(first[k], shared[k]), f"work sharing changed {k}"
    print(f"[fullsize pos {pos}] token {int(tok)}, last layer experts {first['sel'].tolist()} "
          f"(predicted {first['pred'].tolist()})", flush=True)


# ---------------------------------------------------------------------------
# the last layer of the full tensors against the oracle, stage by stage
# ---------------------------------------------------------------------------

#: (after, through) -> outputs held to 99 % bit-identical (and, second, to
#: one ulp), as the layer-0 stage tests of test_gpu_configs.py hold them
LAST_LAYER_STAGES = {
    (None, "qkv"): (("k_new", "v_new", "q"), ()),          # with opcode 8 (the prediction)
    ("qkv", "reduction"): (("attn_out",), ()),
    ("reduction", "oproj"): (("hidden",), ()),
    ("oproj", "rms_router_upgate"): (("normed", "silu"), ("normed",)),
    ("rms_router_upgate", "downproj"): (("hidden",), ()),
}

#: predictor-logit gap below which opcode 8's pair may legitimately come out
#: in another order (fp32 summation order); the drawn residuals are
#: redrawn until the gaps exceed it
PREDICT_MARGIN = 1e-3


def _stage_id(stage):
    return f"{stage[0] or 'start'}-{stage[1]}"


def _residual(case, seed: int) -> torch.Tensor:
    """A residual N(0, 1), redrawn until the oracle's predictor logits of the
    case's layer separate its top three by PREDICT_MARGIN."""
    g = torch.Generator().manual_seed(seed)
    for _ in range(64):
        x = torch.randn(case.g_cpu.hidden_size, generator=g).to(torch.bfloat16)
        case.residual = x
        gap01, gap12 = case.predictor_margins()
        if min(gap01, gap12) > PREDICT_MARGIN:
            return x
    raise AssertionError("no residual with separated predictor logits")


@pytest.mark.parametrize("pos", [4096, PREFILL_C5], ids=["c4", "c5"])
@pytest.mark.parametrize("stage", list(LAST_LAYER_STAGES), ids=_stage_id)
def test_last_layer_stage_against_oracle(model, pos, stage):
    """Layer 31 of the 32-layer model (its gate/up/down rows 29-31 GiB into
    the expert tensors, its K/V rows past 2 GiB into the caches) against the
    oracle on a one-layer copy of the same weights and cache: each stage
    from the oracle's state, its outputs at the rounding-point bar, the
    barrier row equal, the selected experts exact and, in the first stage,
    opcode 8's predicted pair equal to the oracle's (predictor weights =
    router + N(0, 0.007))."""
    from layer_harness import LayerCase
    from moe_harness import MAX_ULP, MIN_EXACT

    last = model.config.num_hidden_layers - 1
    case = LayerCase(model, last, pos)
    after, through = stage
    for seed in (1, 2):
        x = _residual(case, 1000 * pos + seed)
        case.run(after, through, x)
        err, agr = case.errors(), case.agreement()
        tag = f"layer {last} pos {pos} {_stage_id(stage)}"
        print(f"[{tag}] " + " ".join(f"{k} {v:.1e}" for k, v in err.items()), flush=True)
        print(f"[{tag}] ulp/exact " + " ".join(f"{k} {u}/{e:.4f}" for k, (u, e) in agr.items()), flush=True)
        keys, one_ulp = LAST_LAYER_STAGES[stage]
        for k, v in err.items():
            assert v <= 2e-2, f"{tag} {k}: max-abs-rel {v:.3e}"
        for k in keys:
            ulp, exact = agr[k]
            if k in one_ulp:
                assert ulp <= MAX_ULP, f"{tag} {k}: {ulp} ulps"
            assert exact >= MIN_EXACT, f"{tag} {k}: {exact:.4f} bit-identical"
        assert case.barriers_equal(), f"{tag}: barrier tensor differs"
        gi = case.g_gpu.selected_expert_indices.cpu().tolist()
        ri = case.g_cpu.selected_expert_indices.tolist()
        if through in ("rms_router_upgate", "downproj"):
            gap01, gap12 = case.router_margins()
            if min(gap01, gap12) > PREDICT_MARGIN:  # else fp32 summation order may swap a near-tie
                assert gi == ri, f"{tag}: experts {gi} != oracle {ri}"
            else:
                print(f"[{tag}] router near-tie {gap01:.2e} {gap12:.2e}: experts {gi} oracle {ri}", flush=True)
        if after is None:
            gp = case.g_gpu.predicted_expert_indices.cpu().tolist()
            rp = case.g_cpu.predicted_expert_indices.tolist()
            print(f"[{tag}] predicted {gp} oracle {rp} margins {case.predictor_margins()}", flush=True)
            assert gp == rp, f"{tag}: predicted {gp} != oracle {rp}"
