"""Pins for the oracle's attention-side and LM-head solvers
(oracle/python_vm.py, restating megakernels/mixtral/python_vm.py:61-222,
321-345): closed forms, fp64 brute force, invariances, and a whole decode
step against an independent fp64 textbook forward."""

import math

import numpy as np
import pytest
import torch

from megakernels_amd.mixtral.instructions import Mixtral_OProj, Mixtral_RMS_LM_Head
from megakernels_amd.mixtral.scheduler import make_dag, make_globals
from megakernels_amd.mixtral.synthetic import SMALL, TINY, make_synthetic_mixtral, rope_tables, with_layers
from megakernels_amd.scheduler import Schedule
from oracle import python_vm as oracle

BF16 = torch.bfloat16


def test_rope_tables_closed_form():
    cos, sin = rope_tables(50, 64, 10000.0)
    assert torch.allclose(cos * cos + sin * sin, torch.ones_like(cos), atol=1e-6)
    assert torch.equal(cos[0], torch.ones(64)) and torch.equal(sin[0], torch.zeros(64))
    assert torch.equal(cos[:, 0::2], cos[:, 1::2])
    for i in (0, 5, 31):
        ang = 7 * 10000.0 ** (-2 * i / 64)
        assert cos[7, 2 * i].item() == pytest.approx(math.cos(ang), abs=1e-6)
        assert sin[7, 2 * i + 1].item() == pytest.approx(math.sin(ang), abs=1e-6)


def test_rope_is_a_rotation_with_the_reference_sign():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, generator=g).to(BF16)
    cos, sin = rope_tables(100, 64, 1e4)
    y = oracle.rope_interleaved(x, cos[37], sin[37])
    xd, c, s = x.double(), cos[37].double(), sin[37].double()
    # complex form: (x0 + i x1) e^{i theta}
    z = torch.complex(xd[0::2], xd[1::2]) * torch.complex(c[0::2], s[0::2])
    assert torch.allclose(y[0::2].double(), z.real, atol=1e-5)
    assert torch.allclose(y[1::2].double(), z.imag, atol=1e-5)
    # position 0 is the identity; rotations compose (angle addition)
    assert torch.equal(oracle.rope_interleaved(x, cos[0], sin[0]), x.float())
    y2 = oracle.rope_interleaved(y.to(BF16), cos[11], sin[11]).double()
    y3 = oracle.rope_interleaved(x, cos[48], sin[48]).double()
    assert torch.allclose(y2, y3, atol=0.05)


def _fp64_attention(q, k, v, scale):
    s = (q.double() @ k.double().T) * scale
    p = torch.softmax(s, dim=-1)
    return torch.log2(torch.exp(s).sum(-1)), p @ v.double()


def test_attention_partial_against_fp64():
    g = torch.Generator().manual_seed(1)
    q = torch.randn(4, 64, generator=g).to(BF16)
    k = torch.randn(37, 64, generator=g).to(BF16)
    v = torch.randn(37, 64, generator=g).to(BF16)
    lse, out = oracle.attention_partial(q, k, v, 1 / 8)
    lse64, out64 = _fp64_attention(q, k, v, 1 / 8)
    assert torch.allclose(lse.double(), lse64, atol=1e-5)
    assert torch.allclose(out.double(), out64, atol=1e-5)
    lse0, out0 = oracle.attention_partial(q, k[:0], v[:0], 1 / 8)
    assert torch.all(torch.isinf(lse0) & (lse0 < 0)) and not out0.any()


@pytest.mark.parametrize("seq_len,parts", [(1, 1), (17, 3), (100, 7), (33, 8), (5, 4)])
def test_partitions_cover_and_combine(seq_len, parts):
    ranges = [oracle.partial_token_range(seq_len, 16, parts, p) for p in range(parts)]
    toks = [t for a, b in ranges for t in range(a, b)]
    assert toks == list(range(seq_len))
    g = torch.Generator().manual_seed(seq_len)
    q = torch.randn(4, 32, generator=g).to(BF16)
    k = torch.randn(seq_len, 32, generator=g).to(BF16)
    v = torch.randn(seq_len, 32, generator=g).to(BF16)
    lses, outs = zip(*(oracle.attention_partial(q, k[a:b], v[a:b], 0.2) for a, b in ranges))
    _, reduced = oracle.combine_partials(torch.stack(lses, 1), torch.stack(outs, 1))
    _, whole = oracle.attention_partial(q, k, v, 0.2)
    assert torch.allclose(reduced, whole, atol=1e-5)


def _full(config, layers=None, seed=3, prefill=9):
    cfg = with_layers(config, layers) if layers else config
    model = make_synthetic_mixtral(cfg, "cpu", seed, full=True, kv_positions=prefill + 4, prefill=prefill,
                                   ln_weight_std=0.1)
    g = make_globals(model, sm_count=16, seq_len=prefill)
    g.pos_id = prefill
    return model, g


def _textbook_step(model, token, pos):
    """One decode step of the stacked model in fp64 (RMSNorm, QKV, interleaved
    RoPE, GQA attention over the cache plus the new position, O-proj,
    top-2 MoE, final norm and LM head) -- megakernels/mixtral/model.py:60-198
    semantics with no intermediate rounding."""
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
        x = rms(h, sp.ffn_ln_weight[layer])
        logits = sp.router_weight[layer].double() @ x
        top = torch.topk(torch.softmax(logits, 0), 2)
        w = top.values / top.values.sum()
        for j, e in enumerate(top.indices.tolist()):
            gte = sp.expert_gate[layer, e].double() @ x
            upe = sp.expert_up[layer, e].double() @ x
            h = h + w[j] * (sp.expert_down[layer, e].double() @ (torch.nn.functional.silu(gte) * upe))
    out = model.lm_head.lm_head.weight.double() @ rms(h, model.lm_head.input_norm.weight)
    return h, out, kc, vc


def _oracle_step(model, g, token, pos):
    g.hidden_states.copy_(model.embed_tokens[token])
    g.barriers.zero_()
    g.logits.zero_()
    g.pos_id = pos
    nodes, end = make_dag(g)
    oracle.interpret_with_pyvm(g, Schedule(g, nodes, end).get_linear_instructions())


@pytest.mark.parametrize("config,layers", [(SMALL, 2), (TINY, 2)])
def test_decode_step_against_fp64_textbook(config, layers):
    model, g = _full(config, layers)
    pos = g.pos_id
    h64, logits64, kc64, vc64 = _textbook_step(model, 5, pos)
    _oracle_step(model, g, 5, pos)
    rel = lambda a, b: float((a.double() - b).abs().max() / b.abs().max())  # noqa: E731
    assert rel(g.hidden_states, h64) < 3e-2
    assert rel(g.k_cache[:, 0, pos], kc64[:, 0, pos]) < 2e-2
    assert rel(g.v_cache[:, 0, pos], vc64[:, 0, pos]) < 2e-2
    if config.hidden_size >= 2048:
        assert rel(g.logits, logits64) < 3e-2
        assert int(g.logits.float().argmax()) == int(logits64.argmax()) or \
            float(logits64.max() - logits64[int(g.logits.float().argmax())]) < 0.05 * float(logits64.abs().max())
    else:
        assert not g.logits.any()  # no LM head below H = 2048 (2048-column reduction blocks)


def test_barriers_after_a_full_step():
    model, g = _full(TINY, 2)
    _oracle_step(model, g, 1, g.pos_id)
    bars = g.barriers
    bph = g.head_dim // g.qkv_block_size
    heads = g.num_attention_heads + 2 * g.num_kv_heads
    assert torch.all(bars[:, 0, :heads] == bph)
    assert torch.all(bars[:, Mixtral_OProj.opcode() - 1, 0] == g.hidden_size // g.o_proj_block_size)
    assert torch.all(bars[:, 5, 0] == 2 * g.hidden_size // g.down_proj_block_size)


def test_oproj_and_lm_head_closed_forms():
    model, g = _full(TINY, 2)
    gg = torch.Generator().manual_seed(4)
    g.attn_out.copy_(torch.randn(g.attn_out.shape, generator=gg).to(BF16))
    h0 = torch.randn(g.hidden_size, generator=gg).to(BF16)
    g.hidden_states.copy_(h0)
    g.barriers[1, 2, 0] = g.num_attention_heads
    oracle.solve_oproj(g, Mixtral_OProj(1, 3, 4, 0))
    r = slice(3 * g.o_proj_block_size, 4 * g.o_proj_block_size)
    o = (g.o_proj_weights[1][r].double() @ g.attn_out.double()).float().to(BF16)
    assert torch.equal(g.hidden_states[r], (h0[r].float() + o.float()).to(BF16)) or \
        float((g.hidden_states[r].float() - (h0[r].float() + o.float())).abs().max()) <= 2 ** -6 * float(h0.abs().max())
    keep = torch.ones(g.hidden_size, dtype=torch.bool)
    keep[r] = False
    assert torch.equal(g.hidden_states[keep], h0[keep])
    # LM head: the two 2048-column blocks add up to the full matvec
    g.barriers[1, 5, 0] = 2 * g.hidden_size // g.down_proj_block_size
    g.logits.zero_()
    for rb in range(g.hidden_size // 2048):
        oracle.solve_lm_head(g, Mixtral_RMS_LM_Head(0, g.vocab_size // g.lm_head_block_size, rb))
    normed = oracle.rms_norm(g.hidden_states, g.lm_head_norm_weights, g.rms_norm_eps)
    full = g.lm_head_weights.double() @ normed.double()
    err = (g.logits.double() - full).abs().max() / full.abs().max()
    assert float(err) < 1e-2


@pytest.mark.parametrize("config,layers", [(SMALL, 2), (TINY, 2)])
def test_torch_backend_matches_c_backend(config, layers):
    """The oracle's torch backend (the reference's own CPU arithmetic: bf16
    einsum per 16-row block, the RMS norm as torch expressions) against the
    C backend on one whole decode step: same experts and barrier tensor,
    every output within max-abs-rel 2e-2 (after two layers, attention over
    the cache spreads the one-ulp differences of the two summation orders),
    and both held to the fp64 textbook step.  The single MoE layer is held
    to the bit-level bar in test_oracle.py."""
    from moe_harness import max_abs_rel

    out = {}
    try:
        for backend in ("c", "torch"):
            oracle.set_backend(backend)
            model, g = _full(config, layers)
            _oracle_step(model, g, 7, g.pos_id)
            pos = g.pos_id
            out[backend] = {"hidden": g.hidden_states.clone(), "k": g.k_cache[:, 0, pos].clone(),
                            "v": g.v_cache[:, 0, pos].clone(), "q": g.post_ln_rope_q.clone(),
                            "attn": g.attn_out.clone(), "silu": g.expert_silu_out.clone(),
                            "normed": g.router_normed_hidden.clone(), "logits": g.logits.clone(),
                            "sel": g.selected_expert_indices.clone(), "bar": g.barriers.clone()}
            h64, _, _, _ = _textbook_step(model, 7, pos)
            assert float((g.hidden_states.double() - h64).abs().max() / h64.abs().max()) < 3e-2, backend
    finally:
        oracle.set_backend("c")
    c, t = out["c"], out["torch"]
    assert torch.equal(c["sel"], t["sel"]) and torch.equal(c["bar"], t["bar"])
    for k in ("hidden", "k", "v", "q", "attn", "silu", "normed", "logits"):
        if not c[k].any():
            continue
        assert max_abs_rel(t[k], c[k]) <= 2e-2, k


def test_torch_backend_is_selected_explicitly():
    assert oracle.get_backend() == "c"
    with pytest.raises(ValueError):
        oracle.set_backend("numpy")
