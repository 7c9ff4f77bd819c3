"""mk_mixtral_launch_noalloc (no reference counterpart: the launch for
callers that cannot allocate) against mk_mixtral_launch, through the C ABI.

Two calls in a row on one device, the second with a smaller input:

1. a whole-model launch (all opcodes, 8 experts: the config-4 kernel) of a
   two-layer slice of the Mixtral-8x7B shape over 256 workers, with the
   argmax inside the launch -- its scratch holds the exit counter, the
   work-sharing cursors and the spread layer counters;
2. one MoE layer of config 1 (MoE-only kernel) over 64 workers.

Each is run from the same state through both entry points; the Mixtral path
adds in a fixed order, so every output (residual, K/V rows, q, attention
output, logits, SiLU rows, selections, predicted experts, barrier tensor,
token) must be bit-identical.  A queue too large for the fixed scratch is
rejected on the host with MK_ERR_SCRATCH_TOO_SMALL, without a launch.
"""

import ctypes

import pytest
import torch

import mk_mixtral
from megakernels_amd.mixtral.mk import interpret_with_mk
from megakernels_amd.mixtral.scheduler import make_dag, make_globals, make_moe_dag, prefill_oproj_barrier
from megakernels_amd.mixtral.synthetic import C1, C4, make_residuals, make_synthetic_mixtral, with_layers
from megakernels_amd.scheduler import Schedule, assign_to_sms, tensorize_instructions

pytestmark = pytest.mark.gpu

#: tensors of MixtralGlobals a launch writes
OUTPUTS = ("hidden_states", "post_ln_rope_q", "attn_out", "attn_out_intermediates", "attn_lse_intermediates",
           "expert_silu_out", "router_normed_hidden", "logits", "selected_expert_indices",
           "selected_expert_scores", "predicted_expert_indices", "barriers", "k_cache", "v_cache")


def launch_noalloc(*args, stream=None, debug_sync: bool = False, **kwargs):
    """The mk_mixtral callable, launched through mk_mixtral_launch_noalloc."""
    lib = mk_mixtral.load_library()
    g = mk_mixtral.build_globals_struct(*args, **kwargs)
    dev = args[17].device
    with torch.cuda.device(dev):
        s = stream if stream is not None else torch.cuda.current_stream(dev)
        rc = lib.mk_mixtral_launch_noalloc(ctypes.byref(g), ctypes.c_void_p(s.cuda_stream))
        if rc:
            raise mk_mixtral.MKError(rc, lib.mk_mixtral_error_string(rc).decode())
        if debug_sync:
            mk_mixtral.raise_if_failed(dev)


def snapshot(g):
    return {n: getattr(g, n).clone() for n in OUTPUTS}


def restore(g, state):
    for n, t in state.items():
        getattr(g, n).copy_(t)


def run_both(g, tag, want_token: bool = False):
    """The launch from the same state through both entry points; returns the
    outputs of each (and the in-launch argmax token with ``want_token``)."""
    start = snapshot(g)
    outs = []
    for name, fn in (("launch", mk_mixtral.mk_mixtral), ("noalloc", launch_noalloc)):
        restore(g, start)
        torch.cuda.synchronize()
        print(f"[no-alloc] {tag}: {name}", flush=True)
        tok = torch.full((), -1, dtype=torch.long, device=g.hidden_states.device) if want_token else None
        interpret_with_mk(g, fn, debug_sync=True, argmax_out=tok)
        torch.cuda.synchronize()
        out = {n: t.cpu() for n, t in snapshot(g).items()}
        if tok is not None:
            out["token"] = tok.cpu()
        outs.append(out)
    return outs


def assert_identical(tag, a, b):
    for n in a:
        assert torch.equal(a[n], b[n]), f"{tag}: {n} differs between mk_mixtral_launch and the no-alloc launch"


def whole_model_case(workers: int):
    cfg = with_layers(C4, 2)
    model = make_synthetic_mixtral(cfg, "cuda", 31, full=True, kv_positions=4100, prefill=4096,
                                   predictor_sigma=0.007)
    g = make_globals(model, sm_count=workers, seq_len=4096)
    g.pos_id = 4096
    nodes, end = make_dag(g)
    tensorize_instructions(g, assign_to_sms("rr", schedule=Schedule(g, nodes, end)))
    g.hidden_states.copy_(model.embed_tokens[777])
    g.barriers.zero_()
    g.logits.zero_()
    return g


def moe_case(workers: int):
    model = make_synthetic_mixtral(C1, "cuda", 5)
    g = make_globals(model, sm_count=workers)
    nodes, end = make_moe_dag(g)
    tensorize_instructions(g, assign_to_sms("rr", schedule=Schedule(g, nodes, end)))
    g.hidden_states.copy_(make_residuals(1, C1.hidden_size, seed=9, device="cuda")[0])
    g.barriers.zero_()
    prefill_oproj_barrier(g)
    return g


def test_noalloc_matches_launch_twice_second_smaller():
    mk_mixtral.clear_status(0)
    g = whole_model_case(256)
    print(f"[no-alloc] whole model: queues {tuple(g.instructions.shape)}", flush=True)
    a, b = run_both(g, "whole model, 256 workers", want_token=True)
    assert_identical("whole model", a, b)
    assert int(a["token"]) == int(torch.argmax(a["logits"]))
    del g
    torch.cuda.empty_cache()

    g = moe_case(64)
    print(f"[no-alloc] MoE layer: queues {tuple(g.instructions.shape)}", flush=True)
    a, b = run_both(g, "MoE layer, 64 workers")
    assert_identical("MoE layer", a, b)
    assert mk_mixtral.read_status(0)[0] == 0


def test_noalloc_rejects_queues_beyond_its_scratch():
    """2 x 256 x 1100 cursor ints exceed the fixed array: rejected on the
    host (the queues are no-ops; nothing is launched)."""
    g = moe_case(256)
    q = torch.zeros((256, 1100, 32), dtype=torch.int32, device="cuda")
    g.instructions = q
    g.timings = torch.zeros((256, 1100, 128), dtype=torch.int32, device="cuda")
    with pytest.raises(mk_mixtral.MKError) as exc:
        interpret_with_mk(g, launch_noalloc)
    assert exc.value.code == 5, exc.value
    torch.cuda.synchronize()
    # the allocating launch takes the same queues
    interpret_with_mk(g, mk_mixtral.mk_mixtral, debug_sync=True)
