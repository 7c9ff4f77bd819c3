"""In-kernel argmax and next-token embedding (``argmax_out`` /
``next_embed_weights`` of the C ABI).  The reference's generator runs
torch.argmax over the logits and the embedding lookup between launches
(megakernels/generators.py:121-145); here the launch's last workgroup does
both.  Bar: the token equals torch.argmax (CPU) of the logits the same launch
wrote -- also with ties and NaNs planted in the LM head, where torch returns
the first maximal index and counts NaN as maximal -- and hidden_states
becomes exactly that token's embedding row; without ``next_embed_weights``
hidden_states is the layer stack's output, untouched."""

import pytest
import torch

from full_harness import FullCase
from llama_harness import LlamaCase
from megakernels_amd.latency.synthetic import LLAMA_TINY
from megakernels_amd.mixtral.synthetic import TINY
from moe_harness import max_abs_rel

pytestmark = pytest.mark.gpu


def _launch(case, dense: bool, token: int, **kw):
    if dense:
        import mk_llama as mod
        from megakernels_amd.latency.mk import interpret_with_mk

        fn = mod.mk_llama
    else:
        import mk_mixtral as mod
        from megakernels_amd.mixtral.mk import interpret_with_mk

        fn = mod.mk_mixtral
    g = case.g_gpu
    g.hidden_states.copy_(case.gpu_model.embed_tokens[token])
    g.barriers.zero_()
    g.logits.zero_()
    g.pos_id = case.pos
    interpret_with_mk(g, fn, debug_sync=True, **kw)
    torch.cuda.synchronize()


def _plant(w: torch.Tensor, kind: str):
    """Rows of the LM head: 'ties' leaves only +v at rows 3 and 7 and -v at
    rows 4 and 9 (the maximum is then always shared by two rows, or by all
    at 0); 'nan' puts NaN rows at 11 and 20."""
    if kind == "ties":
        v = (torch.randn(w.shape[1], generator=torch.Generator().manual_seed(5)) * 0.05).to(w.dtype).to(w.device)
        w.zero_()
        w[3] = v
        w[7] = v
        w[4] = -v
        w[9] = -v
    elif kind == "nan":
        w[11] = float("nan")
        w[20] = float("nan")


@pytest.mark.parametrize("dense", [False, True], ids=["mixtral", "llama"])
@pytest.mark.parametrize("kind", ["random", "ties", "nan"])
def test_argmax_and_next_embedding(dense, kind):
    case = (LlamaCase(LLAMA_TINY, seed=31, prefill=40, steps=2) if dense
            else FullCase(TINY, seed=31, prefill=40, steps=2))
    _plant(case.g_gpu.lm_head_weights.data, kind)
    out = torch.full((), -1, dtype=torch.long, device="cuda")
    emb = case.gpu_model.embed_tokens
    _launch(case, dense, 9, argmax_out=out, next_embed_weights=emb)
    logits = case.g_gpu.logits.cpu()
    want = int(torch.argmax(logits))
    got = int(out)
    print(f"[argmax {'llama' if dense else 'mixtral'} {kind}] kernel {got} torch {want}", flush=True)
    assert got == want
    if kind == "ties":
        assert want in (0, 3, 4) and int((logits == logits[want]).sum()) >= 2
    if kind == "nan":
        assert want == 11
    assert torch.equal(case.g_gpu.hidden_states.cpu(), emb[want].cpu())


@pytest.mark.parametrize("dense", [False, True], ids=["mixtral", "llama"])
def test_argmax_alone_leaves_hidden(dense):
    case = (LlamaCase(LLAMA_TINY, seed=32, prefill=40, steps=2) if dense
            else FullCase(TINY, seed=32, prefill=40, steps=2))
    _launch(case, dense, 5)
    ref_hidden = case.g_gpu.hidden_states.clone()
    ref_token = int(torch.argmax(case.g_gpu.logits.cpu()))
    out = torch.full((1,), -1, dtype=torch.long, device="cuda")
    _launch(case, dense, 5, argmax_out=out)  # same token and position
    assert int(out[0]) == int(torch.argmax(case.g_gpu.logits.cpu()))
    hidden = case.g_gpu.hidden_states
    if dense:
        # the dense down-projection adds its column chunks into hidden in
        # arrival order, so a relaunch matches to rounding, not bit for bit
        assert max_abs_rel(hidden, ref_hidden) <= 2e-2
        assert int(out[0]) == ref_token or abs(float(case.g_gpu.logits[ref_token]) - float(case.g_gpu.logits.max())) < 0.05
    else:
        assert int(out[0]) == ref_token
        assert torch.equal(hidden, ref_hidden)
    assert not torch.equal(hidden, case.gpu_model.embed_tokens[int(out[0])])


@pytest.mark.parametrize("dense", [False, True], ids=["mixtral", "llama"])
def test_reset_for_next_launch(dense):
    """reset_for_next_launch: the launch ends with the barrier tensor zeroed
    (and the Mixtral logits, which the LM head accumulates); the token is
    the argmax of the logits before the reset, and the next launch, started
    without any fill, gives the same results as one after a fill."""
    case = (LlamaCase(LLAMA_TINY, seed=33, prefill=40, steps=2) if dense
            else FullCase(TINY, seed=33, prefill=40, steps=2))
    g = case.g_gpu
    _launch(case, dense, 11)
    ref_token = int(torch.argmax(g.logits.cpu()))
    ref_hidden = g.hidden_states.clone()
    out = torch.full((), -1, dtype=torch.long, device="cuda")
    _launch(case, dense, 11, argmax_out=out, reset_for_next_launch=True)
    assert int(out) == ref_token
    assert int(g.barriers.abs().sum()) == 0
    if not dense:
        assert not g.logits.any()
    # next launch straight away, no fill: same hidden state as a filled one
    g.hidden_states.copy_(case.gpu_model.embed_tokens[11])
    from megakernels_amd.latency.mk import interpret_with_mk as run_dense
    from megakernels_amd.mixtral.mk import interpret_with_mk as run_moe
    import mk_llama
    import mk_mixtral

    if dense:
        run_dense(g, mk_llama.mk_llama, debug_sync=True)
    else:
        run_moe(g, mk_mixtral.mk_mixtral, debug_sync=True)
    torch.cuda.synchronize()
    if dense:
        assert max_abs_rel(g.hidden_states, ref_hidden) <= 2e-2
    else:
        assert torch.equal(g.hidden_states, ref_hidden)
