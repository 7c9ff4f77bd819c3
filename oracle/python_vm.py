"""CPU oracle for the Mixtral MoE hot path.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` as the checker.  The product
path (``epic-kernel_amd``) never imports it.

A restatement of the reference's Python VM solvers for opcodes 5, 6 and 8:

* ``solve_rms_router_upgate``          megakernels/mixtral/python_vm.py:228-277
* ``solve_expert_downproj_fused``      megakernels/mixtral/python_vm.py:284-314
* ``solve_speculative_expert_predict`` megakernels/mixtral/python_vm.py:356-371
* ``rms_norm`` / matvec helpers        megakernels/demos/latency/python_vm.py:23-56

including the barrier assertions each solver makes before it runs and the
increment it makes after.  The arithmetic of the bf16 matvecs and the RMS
norm is in ``moe_oracle.c`` (same rounding points as torch's bf16 CPU ops);
softmax, top-k and the score renormalisation use torch's fp32 CPU routines,
exactly the calls the reference makes.

Pinning (what keeps this restatement honest, see ``tests/test_oracle.py``):
rounding helpers against torch's own bf16 conversion; ``rms_norm`` against a
literal torch evaluation of the reference expression and closed forms;
matvecs against fp64 brute force; top-2 scores against the closed form
``s0 = 1 / (1 + exp(l1 - l0))``; the full layer against the textbook
``MixtralSparseMoE.forward`` of megakernels/mixtral/model.py:159-198
(different rounding, tolerance only) and against committed golden vectors
produced by an independent torch evaluation (``tests/golden/``).
"""

from __future__ import annotations

import ctypes
import subprocess
import sys
from pathlib import Path

import torch

_HERE = Path(__file__).resolve().parent
_REPO = _HERE.parent
_PKG = _REPO / "epic-kernel_amd"
if str(_PKG) not in sys.path:
    sys.path.insert(0, str(_PKG))

from megakernels_amd.mixtral.instructions import (  # noqa: E402
    ExpertDownProjFused,
    MixtralGlobals,
    RmsRouterUpgate,
    SpeculativeExpertPredict,
)

_LIB_PATH = _HERE / "libmoe_oracle.so"
_lib = None


def build(force: bool = False) -> Path:
    """Compile ``libmoe_oracle.so`` with the committed Makefile."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(_HERE)] + (["-B"] if force else []), check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(str(_LIB_PATH))
        P, I64, F32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float
        L.orc_rms_norm.argtypes = [P, P, I64, F32, P]
        L.orc_router_logits.argtypes = [P, P, I64, I64, P, P]
        L.orc_upgate_silu.argtypes = [P, P, P, I64, I64, I64, P]
        L.orc_down_accumulate.argtypes = [P, P, I64, I64, I64, F32, P]
        L.orc_matvec.argtypes = [P, P, I64, I64, I64, P]
        L.orc_set_num_threads.argtypes = [ctypes.c_int]
        L.orc_get_num_threads.restype = ctypes.c_int
        L.orc_f32_to_bf16.argtypes = [F32]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_bf16_to_f32.restype = F32
        for fn in ("orc_rms_norm", "orc_router_logits", "orc_upgate_silu", "orc_down_accumulate",
                   "orc_matvec", "orc_set_num_threads"):
            getattr(L, fn).restype = None
        _lib = L
    return _lib


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(int(n))


def get_num_threads() -> int:
    return lib().orc_get_num_threads()


def _cpu(t: torch.Tensor, dtype=None) -> torch.Tensor:
    if t.device.type != "cpu":
        raise ValueError("the oracle runs on CPU tensors")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError("the oracle needs contiguous tensors")
    return t


def _p(t: torch.Tensor):
    return ctypes.c_void_p(t.data_ptr())


# ---------------------------------------------------------------------------
# arithmetic helpers
# ---------------------------------------------------------------------------

def rms_norm(inp: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """bf16(weight * bf16(x * rsqrt(mean(x^2) + eps))) -- lat/python_vm.py:50-56."""
    _cpu(inp, torch.bfloat16)
    _cpu(weight, torch.bfloat16)
    out = torch.empty_like(inp)
    lib().orc_rms_norm(_p(inp), _p(weight), inp.numel(), float(eps), _p(out))
    return out


def router_logits(router_w: torch.Tensor, normed: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """``router_w.float() @ normed.float()`` (+ bias) in fp32 -- mkm/python_vm.py:245."""
    _cpu(router_w, torch.bfloat16)
    _cpu(normed, torch.bfloat16)
    E, H = router_w.shape
    out = torch.empty(E, dtype=torch.float32)
    b = None if bias is None else _p(_cpu(bias.float().contiguous()))
    lib().orc_router_logits(_p(router_w), _p(normed), E, H, b, _p(out))
    return out


def matvec(mat: torch.Tensor, vec: torch.Tensor, row0: int = 0, nrows: int | None = None) -> torch.Tensor:
    """bf16 rows ``mat[row0:row0+nrows] @ vec`` -- lat/python_vm.py:29-47."""
    _cpu(mat, torch.bfloat16)
    _cpu(vec, torch.bfloat16)
    nrows = mat.shape[0] - row0 if nrows is None else nrows
    out = torch.empty(nrows, dtype=torch.bfloat16)
    lib().orc_matvec(_p(mat), _p(vec), mat.shape[1], row0, nrows, _p(out))
    return out


def upgate_silu(gate: torch.Tensor, up: torch.Tensor, normed: torch.Tensor, row0: int, nrows: int) -> torch.Tensor:
    """bf16(bf16(silu(bf16(g))) * bf16(u)) for rows of one expert -- mkm/python_vm.py:258-275."""
    for t in (gate, up, normed):
        _cpu(t, torch.bfloat16)
    out = torch.empty(nrows, dtype=torch.bfloat16)
    lib().orc_upgate_silu(_p(gate), _p(up), _p(normed), gate.shape[1], row0, nrows, _p(out))
    return out


def down_accumulate(down: torch.Tensor, act: torch.Tensor, row0: int, nrows: int, score: float,
                    hidden: torch.Tensor) -> None:
    """hidden[r] = bf16(hidden[r] + bf16(score * bf16(down[r] @ act))) -- mkm/python_vm.py:300-310."""
    for t in (down, act, hidden):
        _cpu(t, torch.bfloat16)
    lib().orc_down_accumulate(_p(down), _p(act), down.shape[1], row0, nrows, float(score), _p(hidden))


def select_top_k(logits: torch.Tensor, k: int):
    """softmax -> topk -> renormalise (mkm/python_vm.py:248-250): returns
    (indices int32 [k], fp32 probabilities [k], renormalised fp32 [k])."""
    probs = torch.softmax(logits, dim=-1)
    top, idx = torch.topk(probs, k)
    return idx.to(torch.int32), top, top / top.sum()


# ---------------------------------------------------------------------------
# barrier closed forms (mkm/python_vm.py:38-54)
# ---------------------------------------------------------------------------

def expected_oproj_barrier(globs: MixtralGlobals) -> int:
    return globs.hidden_size // globs.o_proj_block_size


def expected_rms_router_upgate_barrier(globs: MixtralGlobals) -> int:
    return globs.intermediate_size // globs.expert_proj_block_size


def expected_downproj_barrier(globs: MixtralGlobals) -> int:
    return globs.num_experts_per_tok * (globs.hidden_size // globs.down_proj_block_size)


def _bias(globs: MixtralGlobals, layer: int):
    return None if globs.router_bias is None else globs.router_bias[layer]


# ---------------------------------------------------------------------------
# solvers
# ---------------------------------------------------------------------------

def solve_rms_router_upgate(globs: MixtralGlobals, ins: RmsRouterUpgate):
    bar = globs.barriers[ins.layer_idx, ins.prev_opcode() - 1]
    assert bar[0] == expected_oproj_barrier(globs), (
        f"RmsRouterUpgate: expected oproj barrier {expected_oproj_barrier(globs)}, got {int(bar[0])}"
    )
    layer = ins.layer_idx
    normed = rms_norm(globs.hidden_states, globs.ffn_ln_weights[layer], globs.rms_norm_eps)
    globs.router_normed_hidden.copy_(normed)

    logits = router_logits(globs.router_weights[layer], normed, _bias(globs, layer))
    idx, _, scores = select_top_k(logits, globs.num_experts_per_tok)
    globs.selected_expert_indices.copy_(idx)
    globs.selected_expert_scores.copy_(scores.to(globs.selected_expert_scores.dtype))

    bs = globs.expert_proj_block_size
    row0 = ins.start_block_idx * bs
    nrows = ins.num_blocks * bs
    for e in globs.selected_expert_indices.tolist():
        out = upgate_silu(globs.expert_gate_weights[layer, e], globs.expert_up_weights[layer, e], normed, row0, nrows)
        globs.expert_silu_out[e, row0:row0 + nrows] = out

    globs.barriers[layer, ins.opcode() - 1, 0] += ins.num_blocks


def solve_expert_downproj_fused(globs: MixtralGlobals, ins: ExpertDownProjFused):
    bar = globs.barriers[ins.layer_idx, ins.prev_opcode() - 1]
    expected = expected_rms_router_upgate_barrier(globs)
    assert bar[0] == expected, f"ExpertDownProjFused: expected upgate barrier {expected}, got {int(bar[0])}"
    assert ins.reduction_block_idx == 0, "the reduction covers the full intermediate dimension"
    layer = ins.layer_idx
    experts = globs.selected_expert_indices.tolist()
    bs = globs.down_proj_block_size
    row0 = ins.start_block_idx * bs
    nrows = (ins.end_block_idx - ins.start_block_idx) * bs
    for j in range(globs.num_experts_per_tok):
        e = experts[j]
        score = globs.selected_expert_scores[j].float().item()
        down_accumulate(globs.expert_down_weights[layer, e], globs.expert_silu_out[e], row0, nrows, score,
                        globs.hidden_states)
    globs.barriers[layer, ins.opcode() - 1, 0] += (ins.end_block_idx - ins.start_block_idx) * globs.num_experts_per_tok


def solve_speculative_expert_predict(globs: MixtralGlobals, ins: SpeculativeExpertPredict):
    layer = ins.layer_idx
    if layer > 0:
        bar = globs.barriers[layer - 1, ExpertDownProjFused.opcode() - 1]
        assert bar[0] == expected_downproj_barrier(globs)
    normed = rms_norm(globs.hidden_states, globs.ffn_ln_weights[layer], globs.rms_norm_eps)
    weights = globs.router_weights if globs.predictor_weights is None else globs.predictor_weights
    logits = router_logits(weights[layer], normed, _bias(globs, layer))
    idx, _, _ = select_top_k(logits, globs.num_experts_per_tok)
    globs.predicted_expert_indices.copy_(idx)
    globs.barriers[layer, ins.opcode() - 1, 0] += 1


INSTRUCTION_TO_SOLVER = {
    RmsRouterUpgate: solve_rms_router_upgate,
    ExpertDownProjFused: solve_expert_downproj_fused,
    SpeculativeExpertPredict: solve_speculative_expert_predict,
}


def interpret_with_pyvm(globs, instructions, instruction_to_solver=None):
    """Run the linear (topological) instruction list sequentially
    (megakernels/python_vm.py:83-87)."""
    table = INSTRUCTION_TO_SOLVER if instruction_to_solver is None else instruction_to_solver
    for ins in instructions:
        table[type(ins)](globs, ins)


class PyVM_Interpreter:
    def __init__(self, instruction_to_solver=None):
        self.instruction_to_solver = INSTRUCTION_TO_SOLVER if instruction_to_solver is None else instruction_to_solver

    def interpret(self, globs, instructions):
        interpret_with_pyvm(globs, instructions, self.instruction_to_solver)


def moe_layer(hidden, ffn_ln, router_w, gate, up, down, eps, k=2, bias=None):
    """One MoE layer on a single token through the solver arithmetic (all
    rows at once), returning (new_hidden, indices, scores, normed, silu
    [k, F]).  ``gate``/``up`` are [E, F, H], ``down`` [E, H, F]."""
    normed = rms_norm(hidden, ffn_ln, eps)
    logits = router_logits(router_w, normed, bias)
    idx, _, scores = select_top_k(logits, k)
    scores_bf = scores.to(torch.bfloat16)
    F = gate.shape[1]
    silu = torch.stack([upgate_silu(gate[e], up[e], normed, 0, F) for e in idx.tolist()])
    out = hidden.clone()
    for j, e in enumerate(idx.tolist()):
        down_accumulate(down[e], silu[j].contiguous(), 0, down.shape[1], scores_bf[j].float().item(), out)
    return out, idx, scores_bf, normed, silu, logits
