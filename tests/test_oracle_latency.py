"""Pins for the dense (Llama) oracle (oracle/latency_vm.py, restating
megakernels/demos/latency/python_vm.py): closed forms, fp64 brute force, the
column-chunk split of the down projection, and a whole decode step against
an independent fp64 textbook Llama forward."""

import math

import pytest
import torch

from megakernels_amd.latency.instructions import DownProjResidual, LayerNormDoubleMatVecSiLU, RMS_LM_Head
from megakernels_amd.latency.scheduler import expected_downproj_arrivals, make_dag, make_globals
from megakernels_amd.latency.synthetic import LLAMA_SMALL, LLAMA_TINY, make_synthetic_llama, with_layers
from megakernels_amd.scheduler import Schedule
from oracle import latency_vm as lv
from oracle import python_vm as mx

BF16 = torch.bfloat16


def _globals(cfg, layers=None, seed=3, prefill=40, workers=16, **block_sizes):
    cfg = with_layers(cfg, layers) if layers else cfg
    model = make_synthetic_llama(cfg, "cpu", seed, ln_weight_std=0.1, kv_positions=prefill + 4, prefill=prefill)
    g = make_globals(model, seq_len=prefill, sm_count=workers, **block_sizes)
    g.pos_id = prefill
    return model, g


def _rel(a, b):
    return float((a.double() - b).abs().max() / b.abs().max())


def test_upgate_against_fp64_and_its_rounding():
    model, g = _globals(LLAMA_SMALL, layers=1)
    g.hidden_states.copy_(torch.randn(g.hidden_size, generator=torch.Generator().manual_seed(1)).to(BF16))
    g.barriers[0, 3, 0] = lv.expected_oproj_barrier(g)
    blocks = [3, 17, 100]
    lv.solve_upgate(g, LayerNormDoubleMatVecSiLU(0, blocks))
    assert int(g.barriers[0, 4, 0]) == len(blocks)
    x = mx.rms_norm(g.hidden_states, g.mlp_ln_weights[0], g.rms_norm_eps)
    bs = g.up_gate_proj_block_size
    for b in blocks:
        r = slice(b * bs, (b + 1) * bs)
        gt = g.gate_proj_weights[0][r].double() @ x.double()
        up = g.up_proj_weights[0][r].double() @ x.double()
        ref = torch.nn.functional.silu(gt) * up
        assert _rel(g.silu_out[r], ref) < 2e-2
        # the bf16 rounding points: bf16(bf16(silu(bf16 g)) * bf16 u); swapping gate and up fails
        gb, ub = gt.to(BF16), up.to(BF16)
        exact = (torch.nn.functional.silu(gb) * ub)
        assert torch.equal(g.silu_out[r], exact) or _rel(g.silu_out[r], exact.double()) < 1e-2
        swapped = torch.nn.functional.silu(ub) * gb
        assert not torch.allclose(g.silu_out[r].double(), swapped.double(), atol=1e-3)
    untouched = torch.ones(g.intermediate_size, dtype=torch.bool)
    for b in blocks:
        untouched[b * bs:(b + 1) * bs] = False
    assert not g.silu_out[untouched].any()


def test_downproj_column_chunks_add_up_to_the_full_matvec():
    model, g = _globals(LLAMA_SMALL, layers=1, matvec_reduction_size=512)
    gen = torch.Generator().manual_seed(2)
    g.silu_out.copy_(torch.randn(g.intermediate_size, generator=gen).to(BF16))
    h0 = torch.randn(g.hidden_size, generator=gen).to(BF16)
    g.hidden_states.copy_(h0)
    g.barriers[0, 4, 0] = lv.expected_upgate_barrier(g)
    R = g.matvec_reduction_size
    chunks = g.intermediate_size // R
    assert chunks == 4
    for c in range(chunks):
        lv.solve_downproj(g, DownProjResidual(0, 2, 5, c))
    assert int(g.barriers[0, 5, 0]) == chunks * 3
    bs = g.down_proj_block_size
    rows = slice(2 * bs, 5 * bs)
    full = h0[rows].double() + g.down_proj_weights[0][rows].double() @ g.silu_out.double()
    assert _rel(g.hidden_states[rows], full) < 2e-2
    keep = torch.ones(g.hidden_size, dtype=torch.bool)
    keep[rows] = False
    assert torch.equal(g.hidden_states[keep], h0[keep])
    # one chunk alone is the bf16 add of that chunk's bf16 partial
    g.hidden_states.copy_(h0)
    lv.solve_downproj(g, DownProjResidual(0, 2, 3, 1))
    r = slice(2 * bs, 3 * bs)
    part = (g.down_proj_weights[0][r, R:2 * R].double() @ g.silu_out[R:2 * R].double()).to(BF16)
    expect = (h0[r].float() + part.float()).to(BF16)
    assert (g.hidden_states[r].float() - expect.float()).abs().max() <= 2 ** -7 * float(expect.float().abs().max())


def test_lm_head_against_fp64():
    model, g = _globals(LLAMA_TINY, layers=1)
    gen = torch.Generator().manual_seed(4)
    g.hidden_states.copy_(torch.randn(g.hidden_size, generator=gen).to(BF16))
    g.barriers[0, 5, 0] = expected_downproj_arrivals(g)
    lv.solve_lm_head(g, RMS_LM_Head(0, g.vocab_size // g.lm_head_block_size))
    x = mx.rms_norm(g.hidden_states, g.lm_head_norm_weights, g.rms_norm_eps)
    ref = g.lm_head_weights.double() @ x.double()
    assert _rel(g.logits, ref) < 1e-2
    # stored, not accumulated: a second run gives the same logits
    first = g.logits.clone()
    lv.solve_lm_head(g, RMS_LM_Head(0, g.vocab_size // g.lm_head_block_size))
    assert torch.equal(g.logits, first)


def _textbook_step(model, token, pos):
    """One decode step in fp64: RMSNorm, QKV, interleaved RoPE, GQA
    attention over the cache plus the new position, O-proj over all
    columns, SiLU-gated MLP, final norm and LM head (megakernels/llama.py
    semantics, no intermediate rounding)."""
    cfg = model.config
    sp = model.stacked_params
    H, Hq, Hkv, D = cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    eps = cfg.rms_norm_eps

    def rms(x, w):
        return w.double() * x / torch.sqrt((x * x).mean() + eps)

    def rope(x, c, s):
        z = torch.complex(x[0::2], x[1::2]) * torch.complex(c[0::2], s[0::2])
        return torch.stack((z.real, z.imag), -1).reshape(x.shape)

    cos, sin = model.model.rope_cos.double()[pos], model.model.rope_sin.double()[pos]
    h = model.embed_tokens[token].double()
    kc, vc = model.stacked_kv_cache[0].double().clone(), model.stacked_kv_cache[1].double().clone()
    for layer in range(cfg.num_hidden_layers):
        x = rms(h, sp.attn_ln_weight[layer])
        qkv = sp.qkv_proj[layer].double() @ x
        q = qkv[:Hq * D].view(Hq, D)
        k = qkv[Hq * D:(Hq + Hkv) * D].view(Hkv, D)
        v = qkv[(Hq + Hkv) * D:].view(Hkv, D)
        q = torch.stack([rope(q[i], cos, sin) for i in range(Hq)])
        k = torch.stack([rope(k[i], cos, sin) for i in range(Hkv)])
        kc[layer, 0, pos], vc[layer, 0, pos] = k, v
        att = []
        for i in range(Hq):
            kv = i // (Hq // Hkv)
            s = (kc[layer, 0, :pos + 1, kv] @ q[i]) / math.sqrt(D)
            att.append(torch.softmax(s, 0) @ vc[layer, 0, :pos + 1, kv])
        h = h + sp.o_proj[layer].double() @ torch.cat(att)
        x = rms(h, sp.mlp_ln_weight[layer])
        a = torch.nn.functional.silu(sp.gate_proj[layer].double() @ x) * (sp.up_proj[layer].double() @ x)
        h = h + sp.down_proj[layer].double() @ a
    logits = model.lm_head.lm_head.weight.double() @ rms(h, model.lm_head.input_norm.weight)
    return h, logits, kc, vc


@pytest.mark.parametrize("cfg", [LLAMA_SMALL, LLAMA_TINY])
def test_decode_step_against_fp64_textbook(cfg):
    model, g = _globals(cfg, prefill=40)
    pos = g.pos_id
    h64, logits64, kc64, vc64 = _textbook_step(model, 7, pos)
    g.hidden_states.copy_(model.embed_tokens[7])
    nodes, end = make_dag(g)
    lv.interpret_with_pyvm(g, Schedule(g, nodes, end).get_linear_instructions())
    assert _rel(g.hidden_states, h64) < 3e-2
    assert _rel(g.k_cache[:, 0, pos], kc64[:, 0, pos]) < 2e-2
    assert _rel(g.v_cache[:, 0, pos], vc64[:, 0, pos]) < 2e-2
    assert _rel(g.logits, logits64) < 3e-2
    top = int(g.logits.float().argmax())
    assert top == int(logits64.argmax()) or float(logits64.max() - logits64[top]) < 0.05 * float(logits64.abs().max())


def test_oproj_uses_every_attention_column():
    """The reference kernel's O-projection (all Hq * D columns), not lat/
    python_vm.py's first matvec_reduction_size columns: zeroing the columns
    past that prefix must change the result."""
    from megakernels_amd.latency.instructions import O_ProjResidual

    model, g = _globals(LLAMA_SMALL, layers=1, matvec_reduction_size=512)
    assert g.matvec_reduction_size < g.num_attention_heads * g.head_dim
    gen = torch.Generator().manual_seed(5)
    g.attn_out.copy_(torch.randn(g.attn_out.shape, generator=gen).to(BF16))
    h0 = torch.randn(g.hidden_size, generator=gen).to(BF16)
    g.hidden_states.copy_(h0)
    g.barriers[0, 2, 0] = g.num_attention_heads
    mx.solve_oproj(g, O_ProjResidual(0, 0, 1, 0))
    bs = g.o_proj_block_size
    full = h0[:bs].double() + g.o_proj_weights[0][:bs].double() @ g.attn_out.double()
    R = g.matvec_reduction_size
    prefix = h0[:bs].double() + g.o_proj_weights[0][:bs, :R].double() @ g.attn_out[:R].double()
    assert _rel(g.hidden_states[:bs], full) < 2e-2
    assert _rel(g.hidden_states[:bs], prefix) > 5e-2


def test_barriers_after_a_full_step():
    model, g = _globals(LLAMA_SMALL, prefill=300)
    g.hidden_states.copy_(model.embed_tokens[1])
    nodes, end = make_dag(g)
    lv.interpret_with_pyvm(g, Schedule(g, nodes, end).get_linear_instructions())
    bars = g.barriers
    heads = g.num_attention_heads + 2 * g.num_kv_heads
    assert torch.all(bars[:, 0, :heads] == g.head_dim // g.qkv_block_size)
    parts = int(bars[0, 1, 0])
    assert parts > 1 and torch.all(bars[:, 1, :g.num_attention_heads] == parts)
    assert torch.all(bars[:, 2, 0] == g.num_attention_heads)
    assert torch.all(bars[:, 3, 0] == g.hidden_size // g.o_proj_block_size)
    assert torch.all(bars[:, 4, 0] == g.intermediate_size // g.up_gate_proj_block_size)
    assert torch.all(bars[:, 5, 0] == expected_downproj_arrivals(g))
