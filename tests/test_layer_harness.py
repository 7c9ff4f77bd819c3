"""The layer-slice harness of the full-size GPU tests, checked on the CPU:
the oracle running the stages of layer ``l`` of a whole model (the previous
layer's down-projection counter filled) gives exactly what it gives running
the same stages as layer 0 of the harness's one-layer copy of layer ``l``.
So the GPU tests that compare the kernel on layer ``l`` of the full tensors
with the oracle on the copy compare like with like."""

import pytest
import torch

from layer_harness import slice_layer, stage_instructions
from megakernels_amd.latency.synthetic import LLAMA_TINY, make_synthetic_llama
from megakernels_amd.mixtral.synthetic import TINY, make_synthetic_mixtral, with_layers


def _run_both(model, layer, pos, dag_layer, make_globals, prev_done, oracle, dag_kw, stages):
    one = slice_layer(model, layer, "cpu")
    gf = make_globals(model, sm_count=16, seq_len=pos)
    g1 = make_globals(one, sm_count=16, seq_len=pos)
    gf.pos_id = g1.pos_id = pos
    x = torch.randn(gf.hidden_size, generator=torch.Generator().manual_seed(layer)).to(torch.bfloat16)
    for g in (gf, g1):
        g.hidden_states.copy_(x)
        g.barriers.zero_()
        g.logits.zero_()
    gf.barriers[layer - 1, 5, 0] = prev_done(gf)
    for after, through in stages:
        oracle.interpret_with_pyvm(gf, stage_instructions(dag_layer, gf, layer, after, through, **dag_kw))
        oracle.interpret_with_pyvm(g1, stage_instructions(dag_layer, g1, 0, after, through, **dag_kw))
    assert torch.equal(gf.hidden_states, g1.hidden_states)
    assert torch.equal(gf.k_cache[layer], g1.k_cache[0]) and torch.equal(gf.v_cache[layer], g1.v_cache[0])
    assert torch.equal(gf.barriers[layer], g1.barriers[0])
    assert not gf.barriers[layer + 1:].any() and int(gf.barriers[:layer].sum()) == prev_done(gf)
    return gf, g1


def test_mixtral_layer_slice_equals_layer_of_whole_model():
    from megakernels_amd.mixtral.scheduler import expected_downproj_arrivals, make_dag_layer, make_globals
    from oracle import python_vm as oracle

    model = make_synthetic_mixtral(with_layers(TINY, 3), "cpu", 5, full=True, kv_positions=24, prefill=20,
                                   ln_weight_std=0.1, predictor_sigma=0.01)
    stages = [(None, "qkv"), ("qkv", "reduction"), ("reduction", "oproj"), ("oproj", "rms_router_upgate"),
              ("rms_router_upgate", "downproj")]
    gf, g1 = _run_both(model, 2, 20, make_dag_layer, make_globals, expected_downproj_arrivals, oracle,
                       {"predict": True}, stages)
    assert torch.equal(gf.selected_expert_indices, g1.selected_expert_indices)
    assert torch.equal(gf.predicted_expert_indices, g1.predicted_expert_indices)
    assert torch.equal(gf.expert_silu_out, g1.expert_silu_out)
    # a stage list is the difference of two prefixes of the layer's DAG
    full = stage_instructions(make_dag_layer, gf, 2, None, None, predict=True)
    parts = sum((stage_instructions(make_dag_layer, gf, 2, a, t, predict=True) for a, t in stages), [])
    assert parts == full and {i.layer_idx for i in full} == {2}


def test_llama_layer_slice_equals_layer_of_whole_model():
    from dataclasses import replace

    from megakernels_amd.latency.scheduler import expected_downproj_arrivals, make_dag_layer, make_globals
    from oracle import latency_vm as oracle

    model = make_synthetic_llama(replace(LLAMA_TINY, num_hidden_layers=3), "cpu", 6, kv_positions=24, prefill=20)
    stages = [(None, "qkv"), ("qkv", "reduction"), ("reduction", "oproj"), ("oproj", "upgate"),
              ("upgate", "downproj")]
    _run_both(model, 1, 20, make_dag_layer, make_globals, expected_downproj_arrivals, oracle, {}, stages)


def test_stage_instructions_rejects_a_non_prefix():
    from megakernels_amd.mixtral.scheduler import make_dag_layer, make_globals

    model = make_synthetic_mixtral(with_layers(TINY, 2), "cpu", 5, full=True, kv_positions=24, prefill=20)
    g = make_globals(model, sm_count=16, seq_len=20)
    g.pos_id = 20
    with pytest.raises(AssertionError):
        stage_instructions(make_dag_layer, g, 1, "oproj", "qkv")
