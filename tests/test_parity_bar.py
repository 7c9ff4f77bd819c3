"""The GPU parity bar can see a lost bf16 rounding point (CPU only).

The kernel is checked against the oracle with max-abs-rel <= 2e-2 *and* the
rounding-point check of ``moe_harness.assert_bf16_close``: at most one bf16
ulp on normed hidden, and at least 99 % of normed hidden, SiLU and hidden
bit-identical.  Here mistakes a kernel could make are planted in a
copy of the oracle's arithmetic on the CPU (never on the GPU), and the check
must reject each of them while the oracle itself passes:

* RMSNorm rounded once, ``bf16(w * x * r)``, instead of python_vm's
  ``bf16(w * bf16(x * r))`` (lat/python_vm.py:50-56);
* SiLU*up rounded once, ``bf16(silu(g) * u)``, instead of
  ``bf16(bf16(silu(g)) * u)`` (mkm/python_vm.py:258-275);
* SiLU rows read before they were written (a few rows left zero), the
  failure an early opcode-6 read of the overlapped path would cause.

Each planted case also stays within max-abs-rel 2e-2, which is why the
tolerance alone is not the bar.
"""

import pytest
import torch

from megakernels_amd.mixtral.synthetic import C1, make_residuals, make_synthetic_mixtral
from moe_harness import TOL, assert_bf16_close, bf16_agreement, max_abs_rel
from oracle import python_vm as oracle


@pytest.fixture(scope="module")
def layer():
    model = make_synthetic_mixtral(C1, "cpu", seed=7, ln_weight_std=0.1)
    sp = model.stacked_params
    x = make_residuals(1, C1.hidden_size, generator=model.generator)[0]
    return model, sp, x


def _single_rounded_rms(x, w, eps):
    xf = x.float()
    r = torch.rsqrt(xf.pow(2).mean() + eps)
    return (w.float() * (xf * r)).to(torch.bfloat16)


def test_ordinal_distance_counts_representable_steps():
    a = torch.tensor([1.0, -1.0, 0.0, 3.0], dtype=torch.bfloat16)
    up = torch.nextafter(a.float(), torch.full_like(a.float(), 1e9)).to(torch.bfloat16)
    # one bf16 step above each value (the fp32 step rounds back, so bump the bits)
    b = (a.view(torch.int16) + torch.tensor([1, -1, 1, 1], dtype=torch.int16)).view(torch.bfloat16)
    assert bf16_agreement(a, a) == (0, 1.0)
    assert bf16_agreement(b, a) == (1, 0.0)
    # +0 and -0 are the same point; the smallest subnormals on either side are 2 apart
    z = torch.tensor([0.0, -0.0], dtype=torch.bfloat16)
    assert bf16_agreement(z, z.flip(0)) == (0, 1.0)
    tiny = torch.tensor([2 ** -133], dtype=torch.bfloat16)
    assert bf16_agreement(tiny, -tiny)[0] == 2
    del up


def test_oracle_passes_its_own_bar(layer):
    model, sp, x = layer
    eps = C1.rms_norm_eps
    ref = oracle.moe_layer(x, sp.ffn_ln_weight[0], sp.router_weight[0], sp.expert_gate[0], sp.expert_up[0],
                           sp.expert_down[0], eps)
    again = oracle.moe_layer(x, sp.ffn_ln_weight[0], sp.router_weight[0], sp.expert_gate[0], sp.expert_up[0],
                             sp.expert_down[0], eps)
    for a, b in zip(again[:1] + again[3:5], ref[:1] + ref[3:5]):
        assert_bf16_close("oracle", a, b)


def test_single_rounded_rmsnorm_fails(layer):
    model, sp, x = layer
    w = sp.ffn_ln_weight[0]
    ref = oracle.rms_norm(x, w, C1.rms_norm_eps)
    bad = _single_rounded_rms(x, w, C1.rms_norm_eps)
    assert max_abs_rel(bad, ref) <= TOL  # invisible to the tolerance
    with pytest.raises(AssertionError, match="bit-identical"):
        assert_bf16_close("normed", bad, ref)


def test_single_rounded_silu_fails(layer):
    model, sp, x = layer
    normed = oracle.rms_norm(x, sp.ffn_ln_weight[0], C1.rms_norm_eps)
    e = 3
    ref = oracle.upgate_silu(sp.expert_gate[0, e], sp.expert_up[0, e], normed, 0, C1.intermediate_size)
    g = oracle.matvec(sp.expert_gate[0, e].contiguous(), normed).float()
    u = oracle.matvec(sp.expert_up[0, e].contiguous(), normed).float()
    bad = (torch.nn.functional.silu(g) * u).to(torch.bfloat16)
    assert max_abs_rel(bad, ref) <= TOL
    with pytest.raises(AssertionError, match="bit-identical"):
        assert_bf16_close("silu", bad, ref, max_ulp=None)


def test_silu_rows_read_early_fail(layer):
    """Opcode 6 reading a SiLU column group before every row of it is final:
    16 of 3584 rows of one expert still zero when the down projection reads
    them."""
    model, sp, x = layer
    eps = C1.rms_norm_eps
    hidden, idx, scores, normed, silu, _ = oracle.moe_layer(
        x, sp.ffn_ln_weight[0], sp.router_weight[0], sp.expert_gate[0], sp.expert_up[0], sp.expert_down[0], eps)
    stale = silu.clone()
    stale[0, 512:528] = 0
    bad = x.clone()
    for j, e in enumerate(idx.tolist()):
        oracle.down_accumulate(sp.expert_down[0, e], stale[j].contiguous(), 0, C1.hidden_size,
                               scores[j].float().item(), bad)
    assert max_abs_rel(bad, hidden) <= TOL
    with pytest.raises(AssertionError, match="bit-identical"):
        assert_bf16_close("hidden", bad, hidden, max_ulp=None)
