"""Pins for the CPU oracle (oracle/python_vm.py + oracle/moe_oracle.c).

The reference holds no golden vectors for this path, and its CUDA kernel
cannot run here, so each oracle function is pinned by something that does not
restate it: torch's own conversion and library routines (bf16 rounding,
F.rms_norm, softmax/topk, F.silu), fp64 brute force on small inputs, closed
forms, invariants, the textbook MoE forward of megakernels/mixtral/model.py
:159-198 (different rounding, tolerance only), and the committed golden
fixtures produced by an independent torch evaluation of python_vm
(tests/golden/make_golden.py).
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from golden_util import CASE_NAMES, load_case
from megakernels_amd.mixtral.instructions import ExpertDownProjFused, RmsRouterUpgate, SpeculativeExpertPredict
from megakernels_amd.mixtral.scheduler import make_globals, make_moe_dag, prefill_oproj_barrier
from megakernels_amd.mixtral.synthetic import SMALL, MoEConfig, make_residuals, make_synthetic_mixtral
from megakernels_amd.scheduler import Schedule
from moe_harness import max_abs_rel
from oracle import python_vm as oracle

BF16 = torch.bfloat16


def bf16_ulp_diff(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in bf16 units in the last place (same-sign finite values)."""
    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    return (ia - ib).abs()


def rand_bf16(n, std=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, generator=g) * std).to(BF16)


# ---------------------------------------------------------------------------
# bf16 rounding helpers (moe_oracle.c f2bf/bf2f) vs torch's conversion
# ---------------------------------------------------------------------------

def test_bf16_rounding_matches_torch():
    g = torch.Generator().manual_seed(1)
    vals = torch.cat([
        torch.randn(20000, generator=g) * 10.0 ** torch.randint(-30, 30, (20000,), generator=g).float(),
        torch.tensor([0.0, -0.0, 1.0, -1.0, float("inf"), float("-inf"), 1e-40, -1e-40, 3.4e38]),
        # exact halfway cases: even and odd mantissa neighbours
        torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20, -(1.0 + 3 * 2 ** -8)]),
    ])
    lib = oracle.lib()
    ours = torch.tensor([lib.orc_f32_to_bf16(float(v)) for v in vals], dtype=torch.int32)
    ref = vals.to(BF16).view(torch.int16).to(torch.int32) & 0xFFFF
    assert torch.equal(ours, ref)
    assert lib.orc_f32_to_bf16(float("nan")) == 0x7FC0
    for h in (0x3F80, 0xBF80, 0x0001, 0x7F7F, 0x8000):
        ref_h = torch.from_numpy(np.array([h], dtype=np.uint16).view(np.int16)).view(BF16).float().item()
        assert lib.orc_bf16_to_f32(h) == ref_h


# ---------------------------------------------------------------------------
# rms_norm  (lat/python_vm.py:50-56)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n", [512, 1024, 4096])
def test_rms_norm_matches_torch_functional(n):
    x = rand_bf16(n, 1.0, seed=n)
    w = (1.0 + torch.randn(n, generator=torch.Generator().manual_seed(n + 1)) * 0.2).to(BF16)
    eps = 1e-5
    ours = oracle.rms_norm(x, w, eps)
    # library rms_norm in fp32, then the reference's .to(bf16) and bf16 weight multiply
    ref = w * F.rms_norm(x.float(), (n,), eps=eps).to(BF16)
    d = bf16_ulp_diff(ours, ref)
    assert int(d.max()) <= 1
    assert int((d > 0).sum()) <= max(2, n // 500)


def test_rms_norm_double_rounding_is_visible():
    """bf16(w * bf16(x r)) differs from a single rounding bf16(w x r) on some
    elements; the oracle follows the double rounding."""
    n = 4096
    x = rand_bf16(n, 1.0, seed=5)
    w = torch.full((n,), 3.0, dtype=BF16)
    ours = oracle.rms_norm(x, w, 1e-5)
    xf = x.double()
    r = 1.0 / math.sqrt(float((xf * xf).mean()) + 1e-5)
    single = (3.0 * xf * r).float().to(BF16)
    double = (3.0 * (xf * r).float().to(BF16).double()).float().to(BF16)
    assert int((single != double).sum()) > 0
    assert int(bf16_ulp_diff(ours, double).max()) <= 1
    assert int((ours != double).sum()) <= 8


def test_rms_norm_constant_and_scale_invariance():
    n = 1024
    for c in (0.5, 2.0, -3.0):
        x = torch.full((n,), c, dtype=BF16)
        w = torch.full((n,), 1.5, dtype=BF16)
        out = oracle.rms_norm(x, w, 1e-5)
        nv = torch.tensor(c / math.sqrt(c * c + 1e-5), dtype=torch.float32).to(BF16).float()
        assert torch.all(out == torch.tensor(1.5 * float(nv)).to(BF16))
    # eps = 0: scaling x by a power of two changes nothing
    x = rand_bf16(n, 1.0, seed=9)
    w = (1.0 + torch.randn(n, generator=torch.Generator().manual_seed(3)) * 0.1).to(BF16)
    assert torch.equal(oracle.rms_norm(x, w, 0.0), oracle.rms_norm((x.float() * 8).to(BF16), w, 0.0))


# ---------------------------------------------------------------------------
# router logits, top-2, scores  (mkm/python_vm.py:244-253)
# ---------------------------------------------------------------------------

def test_router_logits_fp64_brute_force():
    E, H = 8, 1024
    wr = (torch.randn(E, H, generator=torch.Generator().manual_seed(2)) * 0.02).to(BF16)
    normed = rand_bf16(H, 1.0, seed=3)
    bias = torch.tensor([0.5, -1.0, 0.0, 2.0, 0.25, 0.0, -0.5, 1.0])
    ref = (wr.double().numpy() @ normed.double().numpy()).astype(np.float32)
    assert np.array_equal(oracle.router_logits(wr, normed).numpy(), ref)
    got = oracle.router_logits(wr, normed, bias).numpy()
    assert np.array_equal(got, (ref + bias.numpy()).astype(np.float32))


def test_top2_scores_closed_form():
    g = torch.Generator().manual_seed(4)
    for _ in range(200):
        logits = torch.randn(8, generator=g) * 2
        idx, _, scores = oracle.select_top_k(logits, 2)
        order = np.argsort(-logits.numpy(), kind="stable")
        assert idx.tolist() == order[:2].tolist()
        l0, l1 = float(logits[order[0]]), float(logits[order[1]])
        s0 = 1.0 / (1.0 + math.exp(l1 - l0))
        sb = scores.to(BF16).float()
        assert abs(float(sb[0]) - s0) <= 2 ** -8 * s0 + 1e-7
        assert abs(float(sb[1]) - (1 - s0)) <= 2 ** -8 * max(1 - s0, 1e-3) + 1e-7
        assert float(scores.sum()) == pytest.approx(1.0, abs=1e-6)


# ---------------------------------------------------------------------------
# up/gate + SiLU  (mkm/python_vm.py:258-275)
# ---------------------------------------------------------------------------

def _fp64_rows(mat, vec, row0, nrows):
    return torch.from_numpy(mat[row0:row0 + nrows].double().numpy() @ vec.double().numpy())


def test_upgate_silu_against_torch_silu():
    F_, H = 256, 512
    g = torch.Generator().manual_seed(6)
    gate = (torch.randn(F_, H, generator=g) * 0.05).to(BF16)
    up = (torch.randn(F_, H, generator=g) * 0.05).to(BF16)
    normed = rand_bf16(H, 1.0, seed=7)
    row0, nrows = 32, 200
    ours = oracle.upgate_silu(gate, up, normed, row0, nrows)
    gb = _fp64_rows(gate, normed, row0, nrows).float().to(BF16)
    ub = _fp64_rows(up, normed, row0, nrows).float().to(BF16)
    ref = (F.silu(gb) * ub).to(BF16)
    d = bf16_ulp_diff(ours, ref)
    assert int(d.max()) <= 1 and int((d > 0).sum()) <= 4
    swapped = (F.silu(ub) * gb).to(BF16)  # gate and up exchanged: must not match
    assert int((ours != swapped).sum()) > nrows // 2


# ---------------------------------------------------------------------------
# down projection + weighted residual add  (mkm/python_vm.py:296-310)
# ---------------------------------------------------------------------------

def test_down_accumulate_closed_forms():
    H, F_ = 128, 512
    g = torch.Generator().manual_seed(8)
    down = (torch.randn(H, F_, generator=g) * 0.05).to(BF16)
    act = rand_bf16(F_, 1.0, seed=9)
    h0 = rand_bf16(H, 1.0, seed=10)

    h = h0.clone()
    oracle.down_accumulate(down, act, 0, H, 0.0, h)
    assert torch.equal(h, h0)  # score 0 leaves the residual unchanged
    h = h0.clone()
    oracle.down_accumulate(down, torch.zeros(F_, dtype=BF16), 0, H, 0.7, h)
    assert torch.equal(h, h0)  # zero activations leave it unchanged

    h = h0.clone()
    oracle.down_accumulate(down, act, 16, 64, 0.3125, h)
    o = _fp64_rows(down, act, 16, 64).float().to(BF16)
    ref = h0.clone()
    ref[16:80] = (h0[16:80].float() + (0.3125 * o.float()).to(BF16).float()).to(BF16)
    assert torch.equal(h[:16], h0[:16]) and torch.equal(h[80:], h0[80:])
    assert int(bf16_ulp_diff(h[16:80], ref[16:80]).max()) <= 1


# ---------------------------------------------------------------------------
# whole layer
# ---------------------------------------------------------------------------

def _textbook_moe(x, sp, eps, k=2):
    """megakernels/mixtral/model.py:159-198 in fp32 (different rounding)."""
    n = F.rms_norm(x.float(), (x.numel(),), eps=eps) * sp.ffn_ln_weight[0].float()
    logits = sp.router_weight[0].float() @ n
    p = torch.softmax(logits, -1)
    top, idx = torch.topk(p, k)
    top = top / top.sum()
    out = x.float().clone()
    for j, e in enumerate(idx.tolist()):
        a = F.silu(sp.expert_gate[0, e].float() @ n) * (sp.expert_up[0, e].float() @ n)
        out += top[j] * (sp.expert_down[0, e].float() @ a)
    return out, idx


def test_layer_against_textbook_forward():
    cfg = MoEConfig(1, 512, 1024, 8, 2, 4, 2, 256)
    model = make_synthetic_mixtral(cfg, "cpu", 21, ln_weight_std=0.1)
    sp = model.stacked_params
    for x in make_residuals(6, cfg.hidden_size, generator=model.generator):
        out, idx, *_ = oracle.moe_layer(x, sp.ffn_ln_weight[0], sp.router_weight[0], sp.expert_gate[0],
                                        sp.expert_up[0], sp.expert_down[0], cfg.rms_norm_eps)
        ref, ref_idx = _textbook_moe(x, sp, cfg.rms_norm_eps)
        assert idx.tolist() == ref_idx.tolist()
        assert max_abs_rel(out, ref) <= 2e-2


@pytest.mark.parametrize("name", CASE_NAMES)
def test_oracle_matches_golden(name):
    arrays, meta, model = load_case(name)
    sp = model.stacked_params
    eps = float(meta["eps"])
    bias = None if sp.router_bias is None else sp.router_bias[0]
    for t in range(arrays["hidden_in"].shape[0]):
        out, idx, scores, normed, silu, logits = oracle.moe_layer(
            arrays["hidden_in"][t], sp.ffn_ln_weight[0], sp.router_weight[0], sp.expert_gate[0],
            sp.expert_up[0], sp.expert_down[0], eps, bias=bias)
        assert idx.tolist() == arrays["indices"][t].tolist()
        assert int(bf16_ulp_diff(scores, arrays["scores"][t]).max()) <= 1
        assert np.allclose(logits.numpy(), arrays["logits"][t].numpy(), rtol=1e-5, atol=1e-6)
        dn = bf16_ulp_diff(normed, arrays["normed"][t])
        assert int(dn.max()) <= 1 and int((dn > 0).sum()) <= 2
        ds = bf16_ulp_diff(silu, arrays["silu"][t])
        assert float((ds > 0).float().mean()) <= 0.01 and max_abs_rel(silu, arrays["silu"][t]) <= 1e-2
        assert max_abs_rel(out, arrays["hidden_out"][t]) <= 1e-2
        assert float((out != arrays["hidden_out"][t]).float().mean()) <= 0.02


# ---------------------------------------------------------------------------
# the PyVM solvers: barrier protocol and partition independence
# ---------------------------------------------------------------------------

def _small_globs(workers, **kw):
    model = make_synthetic_mixtral(SMALL, "cpu", 3, ln_weight_std=0.1)
    return model, make_globals(model, sm_count=workers, **kw)


def test_pyvm_asserts_barriers():
    _, g = _small_globs(4)
    with pytest.raises(AssertionError):
        oracle.solve_rms_router_upgate(g, RmsRouterUpgate(0, 0, 1))  # O-proj barrier not met
    prefill_oproj_barrier(g)
    with pytest.raises(AssertionError):
        oracle.solve_expert_downproj_fused(g, ExpertDownProjFused(0, 0, 1, 0))  # opcode 5 not done


def test_pyvm_partition_independent_and_barrier_counts():
    results = []
    for workers, ebs, dbs in ((4, 16, 16), (7, 8, 4), (256, 4, 16)):
        model, g = _small_globs(workers, expert_proj_block_size=ebs, down_proj_block_size=dbs)
        x = make_residuals(1, SMALL.hidden_size, seed=99)[0]
        g.hidden_states.copy_(x)
        prefill_oproj_barrier(g)
        nodes, end = make_moe_dag(g, predict=True)
        oracle.interpret_with_pyvm(g, Schedule(g, nodes, end).get_linear_instructions())
        assert int(g.barriers[0, 4, 0]) == SMALL.intermediate_size // ebs
        assert int(g.barriers[0, 5, 0]) == 2 * (SMALL.hidden_size // dbs)
        assert int(g.barriers[0, 7, 0]) == 1
        assert g.predicted_expert_indices.tolist() == g.selected_expert_indices.tolist()
        results.append(g.hidden_states.clone())
    assert all(torch.equal(results[0], r) for r in results[1:])


def test_predictor_uses_predictor_weights():
    model = make_synthetic_mixtral(SMALL, "cpu", 5, predictor_sigma=0.5)
    g = make_globals(model, sm_count=4)
    g.hidden_states.copy_(make_residuals(1, SMALL.hidden_size, seed=1)[0])
    oracle.solve_speculative_expert_predict(g, SpeculativeExpertPredict(0))
    sp = model.stacked_params
    normed = oracle.rms_norm(g.hidden_states, sp.ffn_ln_weight[0], SMALL.rms_norm_eps)
    expect, _, _ = oracle.select_top_k(oracle.router_logits(sp.predictor_weight[0], normed), 2)
    assert g.predicted_expert_indices.tolist() == expect.tolist()


def test_matvec_column_block_against_fp64():
    """A 2048-column block of a wider matrix (the LM head's reduction blocks,
    read in place through the row stride) equals the fp64 dot products
    rounded once to bf16 (within one bf16 step, fp32 accumulation), and
    equals the same block copied out first, bit for bit."""
    g = torch.Generator().manual_seed(31)
    w = (torch.randn(64, 6144, generator=g) * 0.02).to(torch.bfloat16)
    v = torch.randn(2048, generator=g).to(torch.bfloat16)
    blk = w[:, 2048:4096]
    assert not blk.is_contiguous()
    got = oracle.matvec(blk, v, 8, 40)
    assert torch.equal(got, oracle.matvec(blk.contiguous(), v, 8, 40))
    ref = (blk[8:48].double() @ v.double()).to(torch.bfloat16)
    diff = (got.float() - ref.float()).abs()
    assert float(diff.max()) <= float(ref.float().abs().max()) * 2 ** -7
    # the wrong block (a transposed or shifted read) does not match
    assert not torch.equal(got, oracle.matvec(w[:, :2048], v, 8, 40))


@pytest.mark.parametrize("H,F", [(1024, 3584), (512, 1024)])
def test_torch_backend_moe_layer_bit_level(H, F):
    """One MoE layer through the oracle's torch backend (the reference's
    own CPU arithmetic: bf16 einsum per 16-row block) and its C backend from
    the same input: same experts and scores, normed hidden, SiLU rows and
    hidden within one bf16 ulp and at least 99 % bit-identical."""
    from moe_harness import bf16_agreement

    g = torch.Generator().manual_seed(H + F)
    E = 8
    x = torch.randn(H, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    R = (0.02 * torch.randn(E, H, generator=g)).to(torch.bfloat16)
    G = (0.02 * torch.randn(E, F, H, generator=g)).to(torch.bfloat16)
    U = (0.02 * torch.randn(E, F, H, generator=g)).to(torch.bfloat16)
    D = (0.02 * torch.randn(E, H, F, generator=g)).to(torch.bfloat16)
    res = {}
    try:
        for backend in ("c", "torch"):
            oracle.set_backend(backend)
            res[backend] = oracle.moe_layer(x, w, R, G, U, D, 1e-5)
    finally:
        oracle.set_backend("c")
    (hc, ic, sc, nc, uc, _), (ht, it, st, nt, ut, _) = res["c"], res["torch"]
    assert torch.equal(ic, it) and torch.equal(sc, st)
    for a, b in ((hc, ht), (nc, nt), (uc, ut)):
        ulp, exact = bf16_agreement(b, a)
        assert ulp <= 1 and exact >= 0.99
