"""CPU oracle for the Mixtral MoE hot path.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` as the checker.  The product
path (``epic-kernel_amd``) never imports it.

A restatement of the reference's Python VM solvers:

* ``solve_qkv``                        megakernels/mixtral/python_vm.py:61-118
* ``solve_partial_attn``               megakernels/mixtral/python_vm.py:125-159
* ``solve_attn_reduction``             megakernels/mixtral/python_vm.py:166-189
* ``solve_oproj``                      megakernels/mixtral/python_vm.py:196-215
* ``solve_rms_router_upgate``          megakernels/mixtral/python_vm.py:228-277
* ``solve_expert_downproj_fused``      megakernels/mixtral/python_vm.py:284-314
* ``solve_lm_head``                    megakernels/mixtral/python_vm.py:321-345
* ``solve_speculative_expert_predict`` megakernels/mixtral/python_vm.py:356-371
* ``rms_norm`` / matvec helpers        megakernels/demos/latency/python_vm.py:23-56

including the barrier assertions each solver makes before it runs and the
increment it makes after.  The arithmetic of the bf16 matvecs and the RMS
norm is in ``moe_oracle.c`` (same rounding points as torch's bf16 CPU ops);
softmax, top-k, the score renormalisation, RoPE and attention use torch's
fp32 CPU routines, exactly the calls the reference makes.

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

import math  # noqa: E402

from megakernels_amd.mixtral.instructions import (  # noqa: E402
    ExpertDownProjFused,
    Mixtral_AttnReduction,
    Mixtral_OProj,
    Mixtral_PartialAttn,
    Mixtral_QKV,
    Mixtral_RMS_LM_Head,
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
        L.orc_matvec.argtypes = [P, I64, P, I64, I64, I64, P]
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
# arithmetic backends
# ---------------------------------------------------------------------------
#
# "c" (the default): the bf16 matvecs and the RMS norm in moe_oracle.c (C +
# OpenMP), with the rounding points of torch's bf16 CPU ops.
# "torch": the reference's own CPU arithmetic, call for call -- einsum of a
# bf16 block of 16 rows with a bf16 vector (lat/python_vm.py:29-47, called
# per block by the solvers of mkm/python_vm.py:258-275 and :296-310), the
# RMS norm as torch expressions (lat/python_vm.py:50-56).  Same rounding
# points, torch's own summation order; used as the CPU baseline that runs
# the way the reference's python_vm does.

_BACKEND = "c"
#: rows per einsum of the torch backend (the reference's expert block size)
TORCH_BLOCK_ROWS = 16


def set_backend(name: str) -> None:
    global _BACKEND
    if name not in ("c", "torch"):
        raise ValueError(f"unknown oracle backend {name!r}")
    _BACKEND = name


def get_backend() -> str:
    return _BACKEND


def _einsum_rows(mat: torch.Tensor, vec: torch.Tensor) -> torch.Tensor:
    return torch.einsum("oi,i->o", mat, vec)


# ---------------------------------------------------------------------------
# arithmetic helpers
# ---------------------------------------------------------------------------

def rms_norm(inp: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """bf16(weight * bf16(x * rsqrt(mean(x^2) + eps))) -- lat/python_vm.py:50-56."""
    _cpu(inp, torch.bfloat16)
    _cpu(weight, torch.bfloat16)
    if _BACKEND == "torch":
        x = inp.to(torch.float32)
        x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
        return weight * x.to(inp.dtype)
    out = torch.empty_like(inp)
    lib().orc_rms_norm(_p(inp), _p(weight), inp.numel(), float(eps), _p(out))
    return out


def router_logits(router_w: torch.Tensor, normed: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """``router_w.float() @ normed.float()`` (+ bias) in fp32 -- mkm/python_vm.py:245."""
    _cpu(router_w, torch.bfloat16)
    _cpu(normed, torch.bfloat16)
    E, H = router_w.shape
    if _BACKEND == "torch":
        out = router_w.float() @ normed.float()
        return out if bias is None else out + bias.float()
    out = torch.empty(E, dtype=torch.float32)
    b = None if bias is None else _p(_cpu(bias.float().contiguous()))
    lib().orc_router_logits(_p(router_w), _p(normed), E, H, b, _p(out))
    return out


def matvec(mat: torch.Tensor, vec: torch.Tensor, row0: int = 0, nrows: int | None = None) -> torch.Tensor:
    """bf16 rows ``mat[row0:row0+nrows] @ vec`` -- lat/python_vm.py:29-47.
    ``mat`` may be a column block of a wider matrix (unit column stride)."""
    if mat.device.type != "cpu" or mat.dtype != torch.bfloat16 or mat.dim() != 2 or mat.stride(1) != 1:
        raise ValueError("matvec needs a CPU bf16 matrix with contiguous rows")
    _cpu(vec, torch.bfloat16)
    nrows = mat.shape[0] - row0 if nrows is None else nrows
    if not 0 <= row0 <= row0 + nrows <= mat.shape[0] or vec.numel() != mat.shape[1]:
        raise ValueError("matvec: rows or vector length out of range")
    if _BACKEND == "torch":
        return _einsum_rows(mat[row0:row0 + nrows], vec)
    out = torch.empty(nrows, dtype=torch.bfloat16)
    lib().orc_matvec(_p(mat), mat.stride(0), _p(vec), mat.shape[1], row0, nrows, _p(out))
    return out


def upgate_silu(gate: torch.Tensor, up: torch.Tensor, normed: torch.Tensor, row0: int, nrows: int) -> torch.Tensor:
    """bf16(bf16(silu(bf16(g))) * bf16(u)) for rows of one expert -- mkm/python_vm.py:258-275."""
    for t in (gate, up, normed):
        _cpu(t, torch.bfloat16)
    if _BACKEND == "torch":
        parts = []
        for r in range(row0, row0 + nrows, TORCH_BLOCK_ROWS):
            r1 = min(r + TORCH_BLOCK_ROWS, row0 + nrows)
            g = _einsum_rows(gate[r:r1], normed)
            u = _einsum_rows(up[r:r1], normed)
            parts.append((torch.nn.functional.silu(g) * u).to(torch.bfloat16))
        return torch.cat(parts) if parts else torch.empty(0, dtype=torch.bfloat16)
    out = torch.empty(nrows, dtype=torch.bfloat16)
    lib().orc_upgate_silu(_p(gate), _p(up), _p(normed), gate.shape[1], row0, nrows, _p(out))
    return out


def down_accumulate(down: torch.Tensor, act: torch.Tensor, row0: int, nrows: int, score: float,
                    hidden: torch.Tensor) -> None:
    """hidden[r] = bf16(hidden[r] + bf16(score * bf16(down[r] @ act))) -- mkm/python_vm.py:300-310."""
    for t in (down, act, hidden):
        _cpu(t, torch.bfloat16)
    if _BACKEND == "torch":
        s = torch.tensor(score, dtype=torch.float32)  # the 0-dim fp32 score of mkm/python_vm.py:297
        for r in range(row0, row0 + nrows, TORCH_BLOCK_ROWS):
            r1 = min(r + TORCH_BLOCK_ROWS, row0 + nrows)
            hidden[r:r1] += (s * _einsum_rows(down[r:r1], act)).to(hidden.dtype)
        return
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


# ---------------------------------------------------------------------------
# attention side and LM head (mkm/python_vm.py:61-222, 321-345)
# ---------------------------------------------------------------------------

def rope_interleaved(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Interleaved RoPE of bf16 ``x`` with fp32 ``cos``/``sin`` of the same
    length, returned in fp32: ``x * cos + rot(x) * sin`` with ``rot`` mapping
    the pair (a, b) at (2i, 2i+1) to (-b, a) (``megakernels/llama.py:136-174``;
    bf16 times fp32 promotes to fp32, as in the reference)."""
    rot = torch.stack((-x[1::2], x[0::2]), dim=-1).reshape(x.shape)
    return x * cos + rot * sin


def solve_qkv(globs: MixtralGlobals, ins: Mixtral_QKV):
    """mkm/python_vm.py:61-118."""
    layer = ins.layer_idx
    if layer > 0:
        bar = globs.barriers[layer - 1, ExpertDownProjFused.opcode() - 1]
        assert bar[0] == expected_downproj_barrier(globs), f"QKV layer {layer}: downproj barrier {int(bar[0])}"
    qkv_rope_append(globs, ins)


def qkv_rope_append(globs, ins) -> None:
    """The body of the QKV opcode, shared by the Mixtral and dense VMs
    (mkm/python_vm.py:70-118 = lat/python_vm.py:162-238): RMSNorm with the
    attention norm, bf16 QKV rows, interleaved RoPE on q and k, q to
    ``post_ln_rope_q``, k and v to the caches at ``pos_id``, one arrival per
    block on its head's counter."""
    layer = ins.layer_idx
    post_ln = rms_norm(globs.hidden_states, globs.attn_ln_weights[layer], globs.rms_norm_eps)
    pos = globs.pos_id
    D = globs.head_dim
    k_start = globs.num_attention_heads * D
    v_start = k_start + globs.num_kv_heads * D
    bs = globs.qkv_block_size
    bph = D // bs
    bars = globs.barriers[layer, ins.opcode() - 1]
    for b in range(ins.start_output_block_idx, ins.end_output_block_idx):
        start, end = b * bs, (b + 1) * bs
        out = matvec(globs.qkv_proj_weights[layer], post_ln, start, bs)
        if start < v_start:
            seg = start % D
            out = rope_interleaved(out, globs.rope_cos[pos, seg:seg + bs], globs.rope_sin[pos, seg:seg + bs])
        if start < k_start:
            globs.post_ln_rope_q[start:end] = out.to(torch.bfloat16)
        elif start < v_start:
            s0 = start - k_start
            globs.k_cache[layer, :, pos].view(-1)[s0:s0 + bs] = out.to(torch.bfloat16)
        else:
            s0 = start - v_start
            globs.v_cache[layer, :, pos].view(-1)[s0:s0 + bs] = out
        bars[b // bph] += 1


def attention_partial(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float):
    """(lse [h], out [h, D]) of one split-KV partition in fp32, as
    mkm/python_vm.py:145-149: ``lse = log2(sum(exp(q.k * scale)))``,
    ``out = softmax(q.k * scale) @ v``; an empty partition gives lse = -inf
    and out = 0."""
    qk = (q.float() @ k.float().T) * scale
    lse = torch.log2(torch.sum(torch.exp(qk), dim=-1))
    if k.shape[0] == 0:
        return lse, torch.zeros(q.shape[0], v.shape[-1], dtype=torch.float32)
    return lse, torch.softmax(qk, dim=-1) @ v.float()


def partial_token_range(seq_len: int, kv_block_size: int, num_partials: int, partial_idx: int):
    """Tokens [start, end) of one partition (mkm/python_vm.py:133-140)."""
    total = math.ceil(seq_len / kv_block_size)
    per = math.ceil(total / num_partials)
    b0 = partial_idx * per
    b1 = min(b0 + per, total)
    return b0 * kv_block_size, min(b1 * kv_block_size, seq_len)


def solve_partial_attn(globs: MixtralGlobals, ins: Mixtral_PartialAttn):
    """mkm/python_vm.py:125-159."""
    gqa = globs.num_attention_heads // globs.num_kv_heads
    bph = globs.head_dim // globs.qkv_block_size
    layer, kv = ins.layer_idx, ins.kv_head_idx
    bars = globs.barriers[layer, ins.prev_opcode() - 1]
    for i in range(gqa):
        assert bars[kv * gqa + i] == bph
    assert bars[globs.num_attention_heads + kv] == bph
    assert bars[globs.num_attention_heads + globs.num_kv_heads + kv] == bph
    t0, t1 = partial_token_range(globs.pos_id + 1, globs.attn_kv_block_size, ins.num_partials, ins.partial_idx)
    k = globs.k_cache[layer, 0, t0:t1, kv]
    v = globs.v_cache[layer, 0, t0:t1, kv]
    h0, h1 = kv * gqa, kv * gqa + gqa
    q = globs.post_ln_rope_q.view(globs.num_attention_heads, -1)[h0:h1]
    lse, out = attention_partial(q, k, v, globs.attn_scale)
    if globs.skip_attn_reduction:
        globs.attn_out.view(globs.num_attention_heads, -1)[h0:h1] = out.to(globs.attn_out.dtype)
        globs.barriers[layer, Mixtral_AttnReduction.opcode() - 1, 0] += h1 - h0
    else:
        globs.attn_lse_intermediates[h0:h1, ins.partial_idx] = lse
        globs.attn_out_intermediates[h0:h1, ins.partial_idx] = out
        globs.barriers[layer, ins.opcode() - 1, h0:h1] += 1


def combine_partials(lses: torch.Tensor, outs: torch.Tensor):
    """(denominator [h, 1], reduced [h, D]) of partitions weighted by
    ``2^(lse - max lse)`` (mkm/python_vm.py:176-179)."""
    max_lse = torch.max(lses, dim=-1, keepdim=True).values
    factors = (lses - max_lse).exp2()
    denom = factors.sum(dim=-1, keepdim=True)
    return denom, (outs * factors.unsqueeze(-1)).sum(dim=1) / denom


def solve_attn_reduction(globs: MixtralGlobals, ins: Mixtral_AttnReduction):
    """mkm/python_vm.py:166-189."""
    h0 = ins.head_start_idx
    n = globs.attn_reduction_size
    assert globs.barriers[ins.layer_idx, ins.prev_opcode() - 1, h0] == ins.num_partials
    idx = torch.tensor(ins.reduction_list, dtype=torch.long)
    lses = globs.attn_lse_intermediates[h0:h0 + n, idx]
    outs = globs.attn_out_intermediates[h0:h0 + n, idx]
    denom, reduced = combine_partials(lses, outs)
    if ins.is_terminal:
        globs.attn_out.view(globs.num_attention_heads, -1)[h0:h0 + n] = reduced.to(globs.attn_out.dtype)
    else:
        slot = ins.output_partial_idx
        globs.attn_lse_intermediates[h0:h0 + n, slot] = denom.log().squeeze(-1)
        globs.attn_out_intermediates[h0:h0 + n, slot] = reduced
    globs.barriers[ins.layer_idx, ins.opcode() - 1, 0] += n


def solve_oproj(globs: MixtralGlobals, ins: Mixtral_OProj):
    """mkm/python_vm.py:196-215 with lat/python_vm.py:59-80:
    ``h[rows] = bf16(h[rows] + bf16(W[rows] @ attn_out))``."""
    assert globs.barriers[ins.layer_idx, ins.prev_opcode() - 1, 0] == globs.num_attention_heads
    assert ins.start_block_idx == ins.end_block_idx - 1 and ins.reduction_block_idx == 0
    bs = globs.o_proj_block_size
    r0 = ins.start_block_idx * bs
    out = matvec(globs.o_proj_weights[ins.layer_idx], globs.attn_out, r0, bs)
    globs.hidden_states[r0:r0 + bs] += out
    globs.barriers[ins.layer_idx, ins.opcode() - 1, 0] += ins.end_block_idx - ins.start_block_idx


LM_HEAD_REDUCTION = 2048


def solve_lm_head(globs: MixtralGlobals, ins: Mixtral_RMS_LM_Head):
    """mkm/python_vm.py:321-345: ``logits[rows] += bf16(W[rows, cols] @
    post_ln[cols])`` over the 2048-column block ``reduction_block_idx``."""
    bar = globs.barriers[globs.num_hidden_layers - 1, ExpertDownProjFused.opcode() - 1]
    assert bar[0] == expected_downproj_barrier(globs), f"LM head: downproj barrier {int(bar[0])}"
    post_ln = rms_norm(globs.hidden_states, globs.lm_head_norm_weights.reshape(-1).contiguous(), globs.rms_norm_eps)
    c0 = ins.reduction_block_idx * LM_HEAD_REDUCTION
    cols = slice(c0, c0 + LM_HEAD_REDUCTION)
    w = globs.lm_head_weights[:, cols]
    vec = post_ln[cols].contiguous()
    bs = globs.lm_head_block_size
    for b in range(ins.start_output_block_idx, ins.end_output_block_idx):
        r0 = b * bs
        globs.logits[r0:r0 + bs] += matvec(w, vec, r0, bs)


INSTRUCTION_TO_SOLVER = {
    Mixtral_QKV: solve_qkv,
    Mixtral_PartialAttn: solve_partial_attn,
    Mixtral_AttnReduction: solve_attn_reduction,
    Mixtral_OProj: solve_oproj,
    RmsRouterUpgate: solve_rms_router_upgate,
    ExpertDownProjFused: solve_expert_downproj_fused,
    Mixtral_RMS_LM_Head: solve_lm_head,
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
