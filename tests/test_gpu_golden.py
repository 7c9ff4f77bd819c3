"""The HIP kernel against the committed golden fixtures (tests/golden/), and
the GPU's final barrier tensor against the CPU protocol emulator."""

import pytest
import torch

from golden_util import CASE_NAMES, load_case
from megakernels_amd.mixtral.synthetic import SMALL
from megakernels_amd.protocol import ProtocolDims, simulate
from moe_harness import MoECase, max_abs_rel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", CASE_NAMES)
def test_kernel_matches_golden(name):
    arrays, meta, _ = load_case(name)
    import make_golden

    cfg, seed, ln_std, bias, _ = make_golden.CASES[name]
    case = MoECase(cfg, seed=seed, ln_weight_std=ln_std, router_bias=bias)
    g = case.g_gpu
    for t in range(arrays["hidden_in"].shape[0]):
        case.reset(arrays["hidden_in"][t])
        case.run_gpu()
        idx = g.selected_expert_indices.cpu()
        assert idx.tolist() == arrays["indices"][t].tolist(), f"token {t}"
        sc = g.selected_expert_scores.cpu().view(torch.int16).int()
        assert int((sc - arrays["scores"][t].view(torch.int16).int()).abs().max()) <= 1
        assert max_abs_rel(g.router_normed_hidden, arrays["normed"][t]) <= 2e-2
        silu = g.expert_silu_out.cpu()[idx.long()]
        assert max_abs_rel(silu, arrays["silu"][t]) <= 2e-2
        err = max_abs_rel(g.hidden_states, arrays["hidden_out"][t])
        assert err <= 2e-2, f"token {t}: hidden max-abs-rel {err:.3e}"


@pytest.mark.parametrize("mode", ["rr", "dag"])
def test_gpu_barriers_match_protocol_emulator(mode):
    case = MoECase(SMALL, seed=2, predict=True, mode=mode, workers=16)
    g = case.g_gpu
    x = torch.randn(SMALL.hidden_size, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    case.reset(x)
    start = g.barriers.clone()
    case.run_gpu()
    expect = simulate(g.instructions, start, ProtocolDims.from_globals(g))
    assert torch.equal(g.barriers.cpu(), torch.from_numpy(expect).to(torch.int32))
