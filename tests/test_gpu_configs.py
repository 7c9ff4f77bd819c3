"""GPU parity at the exact shapes of BASELINE configs 2-5, against the CPU
oracle (the reference runs its stage harness at the full Mixtral shapes,
demos/mixtral/debug_mixtral_mk_full.py:36-75).

* Configs 3, 4 and 5 run as two-layer slices of their exact shapes, with the
  real vocabulary and LM head and the real cached context:
  - C4: hidden 4096, 32/8 heads, head dim 128, 8 experts, FFN 14336, vocab
    32000, RoPE theta 1e6, 4096 cached positions;
  - C5: the C4 shape with 16384 cached positions and a predictor whose
    weights are the router's plus N(0, 0.007);
  - C3: hidden 3072, 24/8 heads, FFN 8192, vocab 128256, RoPE theta 500000,
    2048 cached positions (the dense VM).
  Each takes three decode steps (the cache grows by one row per step) and
  checks the residual, the new K/V rows, rotated q, the attention output and
  the logits within max-abs-rel 2e-2, the last layer's expert indices (and
  the predicted pair) exactly, and the barrier tensor equal to the oracle's.
  These are whole-model steps: from the second layer on, a stage's inputs
  carry the earlier stages' last-place differences, and attention over
  thousands of random cached positions spreads a few one-ulp differences in
  q to most elements of its output (measured: 30-70 % of the last layer's
  bf16 outputs bit-identical after two layers).  The bit-identical fractions
  are printed, not held to a floor.
* The stage tests start from the oracle's own state (``start_after_op``,
  the reference diff harness's mode), so the stage under test sees
  bit-identical inputs and its outputs are held to the rounding-point bar
  of ``moe_harness`` (at least 99 % bit-identical; normed hidden within one
  ulp when its input is the oracle's).  The LM head is checked the same way
  from the state after the last layer (``downproj``); from earlier stages
  its logits are held to max-abs-rel only, since its RMSNorm reads the
  whole residual, whose few last-place differences move every logit.
* Config 2: one full-size MoE layer, uniform and with the skewed router
  bias, token by token.
"""

import pytest
import torch

from full_harness import FullCase
from llama_harness import LlamaCase
from megakernels_amd.latency.synthetic import C3
from megakernels_amd.mixtral.synthetic import C2, C4, with_layers
from moe_harness import MAX_ULP, MIN_EXACT, MoECase, draw_tokens

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _report(tag, case):
    err = case.errors()
    agr = case.agreement()
    print(f"[{tag}] pos {case.pos - 1} " + " ".join(f"{k} {v:.1e}" for k, v in err.items()), flush=True)
    print(f"[{tag}] ulp/exact " + " ".join(f"{k} {u}/{e:.4f}" for k, (u, e) in agr.items()), flush=True)
    return err, agr


def _check_through(tag, case):
    err, _ = _report(tag, case)
    for k, v in err.items():
        assert v <= TOL, f"{tag} {k}: max-abs-rel {v:.3e}"
    assert case.barriers_equal(), f"{tag}: barrier tensor differs from the oracle's"


#: router-logit gap below which the last layer's selection may legitimately
#: differ from the oracle's after whole-model steps (the residual differs by
#: up to max-abs-rel ~1e-2 there); the layer-only tests draw inputs with a
#: 1e-3 margin instead
TIE_MARGIN = 0.05


def _check_selection(case):
    """The last layer's expert pair equal to the oracle's, in order, unless
    the oracle's top-2 router logits are within TIE_MARGIN (then as a set)
    or its 2nd and 3rd are (then the first expert only).  The predicted pair
    is printed: the pre-attention residual it came from is not kept, so its
    margins are unknown."""
    from oracle import python_vm as oracle

    g, r = case.g_gpu, case.g_cpu
    last = g.num_hidden_layers - 1
    gi, ri = case.indices()
    logits = oracle.router_logits(r.router_weights[last].contiguous(), r.router_normed_hidden)
    top = torch.sort(logits, descending=True).values
    gap01, gap12 = float(top[0] - top[1]), float(top[1] - top[2])
    print(f"[selection] {gi} oracle {ri} gaps {gap01:.3f} {gap12:.3f}; predicted "
          f"{g.predicted_expert_indices.cpu().tolist()} oracle {r.predicted_expert_indices.tolist()}", flush=True)
    if gap12 < TIE_MARGIN:
        assert gi[0] == ri[0] or gap01 < TIE_MARGIN
    elif gap01 < TIE_MARGIN:
        assert sorted(gi) == sorted(ri)
    else:
        assert gi == ri, f"experts {gi} != oracle {ri}"


def _check_prediction(case, tok, margin=1e-3):
    """Opcode 8's predicted pair (layer 0, from the token's embedding) equal
    to the oracle's, in order, unless the oracle's predictor logits are
    within ``margin`` (then as a set, or the first expert only)."""
    from oracle import python_vm as oracle

    r = case.g_cpu
    x = case.cpu_model.embed_tokens[tok].contiguous()
    normed = oracle.rms_norm(x, r.ffn_ln_weights[0], r.rms_norm_eps)
    w = r.router_weights if r.predictor_weights is None else r.predictor_weights
    top = torch.sort(oracle.router_logits(w[0].contiguous(), normed), descending=True).values
    gap01, gap12 = float(top[0] - top[1]), float(top[1] - top[2])
    gp, rp = case.g_gpu.predicted_expert_indices.cpu().tolist(), r.predicted_expert_indices.tolist()
    print(f"[prediction] {gp} oracle {rp} gaps {gap01:.2e} {gap12:.2e}", flush=True)
    if gap12 < margin:
        assert gp[0] == rp[0] or gap01 < margin
    elif gap01 < margin:
        assert sorted(gp) == sorted(rp)
    else:
        assert gp == rp, f"predicted {gp} != oracle {rp}"


def _check_stage(tag, case, exact_keys, one_ulp=()):
    """Every output within max-abs-rel; ``exact_keys`` at least 99 %
    bit-identical; ``one_ulp`` within one bf16 ulp everywhere."""
    err, agr = _report(tag, case)
    for k, v in err.items():
        assert v <= TOL, f"{tag} {k}: max-abs-rel {v:.3e}"
    for k in exact_keys:
        ulp, exact = agr[k]
        if k in one_ulp:
            assert ulp <= MAX_ULP, f"{tag} {k}: {ulp} bf16 ulps from the oracle"
        assert exact >= MIN_EXACT, f"{tag} {k}: {exact:.4f} bit-identical (bar {MIN_EXACT})"
    assert case.barriers_equal(), f"{tag}: barrier tensor differs from the oracle's"


# ---------------------------------------------------------------------------
# configs 4 and 5: two-layer slices of the Mixtral-8x7B shape
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("prefill,sigma", [(4096, None), (16384, 0.007)], ids=["c4", "c5"])
def test_mixtral_two_layers_at_config_shape(prefill, sigma):
    case = FullCase(with_layers(C4, 2), seed=40, prefill=prefill, steps=3, generate_on_device=True,
                    ln_weight_std=0.1, predictor_sigma=sigma)
    parts = max(i.num_partials for i in case.linear if i.opcode() == 2)
    print(f"[c4-shape x2, {prefill} cached] {len(case.linear)} instructions, {parts} partitions per KV head",
          flush=True)
    for tok in (11, 23000, 31999):
        case.step(tok)
        _check_through(f"{'c5' if sigma else 'c4'} x2", case)
        _check_selection(case)


# ---------------------------------------------------------------------------
# config 3: two-layer slice of the Llama-3.2-3B shape (dense VM)
# ---------------------------------------------------------------------------

def test_llama_two_layers_at_config_shape():
    case = LlamaCase(with_layers(C3, 2), seed=41, prefill=2048, steps=3, generate_on_device=True)
    for tok in (5, 64000, 128255):
        case.step(tok)
        _check_through("c3 x2", case)


# ---------------------------------------------------------------------------
# stages from the oracle's state, at the config-4 (and config-3) shapes
# ---------------------------------------------------------------------------

#: one stage at a time, from the oracle's state: (after, through) -> (outputs
#: held to 99 % bit-identical, those also held to one ulp); None: from the
#: start of the step, or through the LM head
MIXTRAL_STAGES = {
    (None, "qkv"): (("k_new", "v_new", "q"), ()),
    ("qkv", "reduction"): (("attn_out",), ()),          # partial attention + LSE reduction
    ("partial", "reduction"): (("attn_out",), ()),      # LSE reduction alone
    ("reduction", "oproj"): (("hidden",), ()),
    ("oproj", "rms_router_upgate"): (("normed", "silu"), ("normed",)),
    ("rms_router_upgate", "downproj"): (("hidden",), ()),  # opcode 6, routing read from memory
    ("downproj", None): (("logits",), ()),               # the LM head
}


def _stage_id(stage):
    return f"{stage[0] or 'start'}-{stage[1] or 'lm_head'}"


@pytest.mark.parametrize("stage", list(MIXTRAL_STAGES), ids=_stage_id)
def test_mixtral_stage_from_oracle_state(stage):
    """One stage of a C4-shaped layer (4096 cached positions, vocab 32000):
    the schedule through ``after`` of layer 0 on the oracle, then the stages
    through ``through`` on the kernel and on the oracle from the same state."""
    after, through = stage
    case = FullCase(with_layers(C4, 1), seed=42, prefill=4096, steps=2, generate_on_device=True,
                    ln_weight_std=0.1, start_after_op=after, stop_after_op=through)
    for tok in (3, 17):
        case.step(tok)
        keys, one_ulp = MIXTRAL_STAGES[stage]
        _check_stage(f"c4 {_stage_id(stage)}", case, keys, one_ulp)
        if through == "rms_router_upgate":
            gi, ri = case.indices()
            assert gi == ri
        if after is None:
            _check_prediction(case, tok)


LLAMA_STAGES = {
    (None, "qkv"): ("k_new", "v_new", "q"),
    ("qkv", "reduction"): ("attn_out",),
    ("reduction", "oproj"): ("hidden",),
    ("oproj", "upgate"): ("silu",),
    ("upgate", "downproj"): ("hidden",),  # full-row down projection, one writer per row
    ("downproj", None): ("logits",),
}


@pytest.mark.parametrize("stage", list(LLAMA_STAGES), ids=_stage_id)
def test_llama_stage_from_oracle_state(stage):
    """One stage of a C3-shaped layer (2048 cached positions, the
    128256-row LM head) on the dense VM, from the oracle's state."""
    after, through = stage
    case = LlamaCase(with_layers(C3, 1), seed=43, prefill=2048, steps=2, generate_on_device=True,
                     start_after_op=after, stop_after_op=through)
    for tok in (9, 100000):
        case.step(tok)
        _check_stage(f"c3 {_stage_id(stage)}", case, LLAMA_STAGES[stage])


# ---------------------------------------------------------------------------
# config 2: one full-size MoE layer, uniform and skewed
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("skewed", [False, True], ids=["uniform", "skewed"])
def test_c2_full_shape_tokens(skewed):
    bias = [2.0, 2.0] + [0.0] * (C2.num_local_experts - 2) if skewed else None
    case = MoECase(C2, seed=44, generate_on_device=True, router_bias=bias, ln_weight_std=0.1)
    hits = 0
    for x in draw_tokens(case.cpu_model, 8):
        res = case.run_token(x)
        print(f"[c2 {'skewed' if skewed else 'uniform'}] experts {res.indices_gpu} hidden {res.err_hidden:.1e} "
              f"ulp/exact normed {res.agree_normed} silu {res.agree_silu} hidden {res.agree_hidden}", flush=True)
        res.assert_ok()
        hits += sum(i in (0, 1) for i in res.indices_ref)
    if skewed:
        assert hits >= 12
