"""``mk_mixtral`` -- the drop-in launcher module.

The reference imports its compiled kernel as ``from mk_mixtral import
mk_mixtral`` after putting the build directory on ``sys.path``
(``megakernels/mixtral/mk.py:100-104``) and calls it with 31 positional
arguments in the field order of ``mixtral_globals``
(``demos/mixtral/mixtral.cu:43-93``) plus ``stream=``.  This module provides
the same callable for the MI355X build: it validates the tensors, fills the
C-ABI struct of ``include/mk_mixtral.h`` and calls ``mk_mixtral_launch`` in
``libmk_mixtral.so`` (built from ``csrc/mk_mixtral.hip``) through ctypes.

Keyword-only additions (defaults reproduce the reference kernel, whose block
sizes are the compile-time 16):

``expert_proj_block_size``, ``down_proj_block_size``, ``o_proj_block_size``
    the ``MixtralGlobals`` block sizes the instructions were built with;
``router_bias`` / ``predictor_weights``
    the optional MoE extensions (see ``include/mk_mixtral.h``);
``spin_timeout_us``
    bound on every in-kernel barrier wait (default 2 s);
``record_timings``
    write per-instruction ``s_memrealtime`` stamps into ``timings``;
``work_sharing``
    let workers that finish their own opcode-5 rows take unclaimed rows of
    other workers' opcode-5 instructions (default off: each instruction
    processes exactly its own rows; results and barrier counts are the same
    either way);
``argmax_out`` / ``next_embed_weights``
    decode-driver extension (whole-model launches): the launch ends by
    writing ``argmax(logits)`` (torch.argmax's first-maximum, NaN-maximal
    order) into the int64 ``argmax_out``, and with the ``[V, H]`` embedding
    table sets ``hidden_states`` to that token's row, the next step's input
    -- what the reference's generator does with torch between launches;
``reset_for_next_launch``
    the launch ends by zeroing the barrier tensor and the logits, so that
    the next launch needs no fill (neither can be read afterwards);
``downproj_overlap``
    opcode 5 also counts finished SiLU rows per 512-row column chunk, and
    opcode 6 starts on groups of chunks as they complete (no counterpart in
    the reference; ignored with ``work_sharing``); meant for an opcode-5
    partition interleaved across workers.  Same indices, scores and barrier
    counts; the hidden state differs only in fp32 summation order;
``late_loads``
    prefetch off: every instruction waits for its inputs before it loads
    anything, and no predicted expert rows are staged (for prefetch on/off
    comparisons; same results);
``debug_sync``
    synchronise after the launch and raise :class:`MKDeviceError` if the
    kernel recorded a failure.

There is no fallback: if the library is missing or the tensors are not on a
GPU, the call raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

__all__ = [
    "mk_mixtral",
    "MKError",
    "MKDeviceError",
    "read_status",
    "clear_status",
    "query_device",
    "library_path",
]

_HERE = Path(__file__).resolve().parent
_LIB_NAME = "libmk_mixtral.so"

ABI_VERSION = 5
STATUS_WORDS = 16
MAX_EXPERTS = 16

_ERROR_NAMES = {
    0: "MK_OK",
    1: "MK_ERR_INVALID_ARGUMENT",
    2: "MK_ERR_UNSUPPORTED",
    3: "MK_ERR_HIP",
    4: "MK_ERR_NOT_CORESIDENT",
    5: "MK_ERR_SCRATCH_TOO_SMALL",
    16: "MK_ERR_TIMEOUT",
    17: "MK_ERR_BAD_OPCODE",
    18: "MK_ERR_UNSUPPORTED_OPCODE",
    19: "MK_ERR_BAD_INSTRUCTION",
}


class MKError(RuntimeError):
    """A host-side failure of ``mk_mixtral_launch``."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{_ERROR_NAMES.get(code, code)}: {message}")
        self.code = code


class MKDeviceError(MKError):
    """A failure the kernel recorded in its status words."""

    def __init__(self, status: list[int], message: str):
        super().__init__(status[0], message)
        self.status = status
        self.worker, self.slot, self.opcode, self.layer, self.expected, self.seen = status[1:7]


_P = ctypes.c_void_p


class MkMixtralGlobals(ctypes.Structure):
    """ctypes mirror of ``mk_mixtral_globals`` (include/mk_mixtral.h)."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("abi_version", ctypes.c_uint32),
        ("barriers", _P),
        ("bar_layers", ctypes.c_int64),
        ("bar_ops", ctypes.c_int64),
        ("bar_width", ctypes.c_int64),
        ("instructions", _P),
        ("num_workers", ctypes.c_int64),
        ("queue_len", ctypes.c_int64),
        ("timings", _P),
        ("qkv_weights", _P),
        ("attn_norm_weights", _P),
        ("o_weights", _P),
        ("expert_gate_weights", _P),
        ("expert_up_weights", _P),
        ("expert_down_weights", _P),
        ("router_weights", _P),
        ("ffn_ln_weights", _P),
        ("lm_head_norm_weights", _P),
        ("lm_head_weights", _P),
        ("k_cache", _P),
        ("v_cache", _P),
        ("rope_cos", _P),
        ("rope_sin", _P),
        ("hidden_states", _P),
        ("q_post_rope", _P),
        ("attn_out", _P),
        ("attn_lse_intermediates", _P),
        ("attn_out_intermediates", _P),
        ("expert_silu_out", _P),
        ("router_normed_hidden", _P),
        ("logits", _P),
        ("selected_expert_indices", _P),
        ("selected_expert_scores", _P),
        ("predicted_expert_indices", _P),
        ("pos_id", ctypes.c_uint32),
        ("attn_scale", ctypes.c_float),
        ("rms_norm_eps", ctypes.c_float),
        ("skip_attn_reduction", ctypes.c_int32),
        ("num_layers", ctypes.c_int32),
        ("hidden_size", ctypes.c_int32),
        ("intermediate_size", ctypes.c_int32),
        ("num_experts", ctypes.c_int32),
        ("num_experts_per_tok", ctypes.c_int32),
        ("expert_proj_block_size", ctypes.c_int32),
        ("down_proj_block_size", ctypes.c_int32),
        ("o_proj_block_size", ctypes.c_int32),
        ("qkv_block_size", ctypes.c_int32),
        ("attn_kv_block_size", ctypes.c_int32),
        ("lm_head_block_size", ctypes.c_int32),
        ("lm_head_reduction", ctypes.c_int32),
        ("num_attention_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("vocab_size", ctypes.c_int32),
        ("kv_capacity", ctypes.c_int32),
        ("attn_partial_slots", ctypes.c_int32),
        ("router_bias", _P),
        ("predictor_weights", _P),
        ("status", _P),
        ("spin_timeout_us", ctypes.c_uint32),
        ("record_timings", ctypes.c_int32),
        ("work_sharing", ctypes.c_int32),
        ("argmax_out", _P),
        ("next_embed_weights", _P),
        ("reset_for_next_launch", ctypes.c_int32),
        ("downproj_overlap", ctypes.c_int32),
        ("late_loads", ctypes.c_int32),
    ]


#: C entry points declared in include/mk_mixtral.h
EXPORTED_SYMBOLS = (
    "mk_mixtral_launch",
    "mk_mixtral_launch_noalloc",
    "mk_mixtral_read_status",
    "mk_mixtral_clear_status",
    "mk_mixtral_query_device",
    "mk_mixtral_error_string",
    "mk_mixtral_last_hip_error",
    "mk_mixtral_last_error_site",
    "mk_mixtral_abi_version",
    "mk_mixtral_reload_overrides",
)

_lib = None


def library_path() -> Path:
    return Path(os.environ.get("MK_MIXTRAL_LIB", _HERE / _LIB_NAME))


def load_library():
    """Load ``libmk_mixtral.so`` (after torch, so the HIP runtime torch
    already loaded is the one the library binds to)."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise MKError(2, f"{path} not found; build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = ctypes.CDLL(str(path))
    lib.mk_mixtral_launch.argtypes = [ctypes.POINTER(MkMixtralGlobals), ctypes.c_void_p]
    lib.mk_mixtral_launch.restype = ctypes.c_int
    lib.mk_mixtral_launch_noalloc.argtypes = [ctypes.POINTER(MkMixtralGlobals), ctypes.c_void_p]
    lib.mk_mixtral_launch_noalloc.restype = ctypes.c_int
    lib.mk_mixtral_read_status.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_int32)]
    lib.mk_mixtral_read_status.restype = ctypes.c_int
    lib.mk_mixtral_clear_status.argtypes = [ctypes.c_int]
    lib.mk_mixtral_clear_status.restype = ctypes.c_int
    lib.mk_mixtral_query_device.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)]
    lib.mk_mixtral_query_device.restype = ctypes.c_int
    lib.mk_mixtral_error_string.argtypes = [ctypes.c_int]
    lib.mk_mixtral_error_string.restype = ctypes.c_char_p
    lib.mk_mixtral_last_hip_error.restype = ctypes.c_int
    lib.mk_mixtral_last_error_site.restype = ctypes.c_char_p
    lib.mk_mixtral_abi_version.restype = ctypes.c_int
    lib.mk_mixtral_reload_overrides.argtypes = []
    lib.mk_mixtral_reload_overrides.restype = None
    if lib.mk_mixtral_abi_version() != ABI_VERSION:
        raise MKError(1, f"{path} has ABI {lib.mk_mixtral_abi_version()}, expected {ABI_VERSION}")
    _lib = lib
    return lib


def _error_text(lib, code: int) -> str:
    text = lib.mk_mixtral_error_string(code).decode()
    if code == 3:
        text += (f" (hipError_t {lib.mk_mixtral_last_hip_error()} from "
                 f"{lib.mk_mixtral_last_error_site().decode()})")
    return text


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _check(cond: bool, msg: str, exc=ValueError):
    if not cond:
        raise exc(msg)


def _check_tensor(name, t, dtype, device, shape=None, min_numel=None):
    _check(isinstance(t, torch.Tensor), f"{name} must be a torch.Tensor", TypeError)
    _check(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}", TypeError)
    _check(t.device == device, f"{name} is on {t.device}, expected {device}")
    _check(t.is_contiguous(), f"{name} must be contiguous")
    if shape is not None:
        _check(tuple(t.shape) == tuple(shape), f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if min_numel is not None:
        _check(t.numel() >= min_numel, f"{name} has {t.numel()} elements, needs >= {min_numel}")


def query_device(device=None) -> tuple[int, int]:
    """(compute units, largest co-resident worker count) of ``device``."""
    lib = load_library()
    dev = torch.device(device if device is not None else "cuda")
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    cus, workers = ctypes.c_int32(), ctypes.c_int32()
    rc = lib.mk_mixtral_query_device(idx, ctypes.byref(cus), ctypes.byref(workers))
    if rc:
        raise MKError(rc, _error_text(lib, rc))
    return cus.value, workers.value


def read_status(device=None) -> list[int]:
    """Synchronise ``device`` and return the kernel's 16 status words."""
    lib = load_library()
    dev = torch.device(device if device is not None else "cuda")
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    buf = (ctypes.c_int32 * STATUS_WORDS)()
    rc = lib.mk_mixtral_read_status(idx, buf)
    if rc:
        raise MKError(rc, _error_text(lib, rc))
    return list(buf)


def clear_status(device=None) -> None:
    lib = load_library()
    dev = torch.device(device if device is not None else "cuda")
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    rc = lib.mk_mixtral_clear_status(idx)
    if rc:
        raise MKError(rc, _error_text(lib, rc))


def raise_if_failed(device=None) -> None:
    """Raise :class:`MKDeviceError` (and clear the status) if a launch on
    ``device`` recorded a failure."""
    st = read_status(device)
    if st[0] != 0:
        lib = load_library()
        clear_status(device)
        raise MKDeviceError(
            st,
            f"{_error_text(lib, st[0])} at worker {st[1]} slot {st[2]} opcode {st[3]} "
            f"layer {st[4]} (expected {st[5]}, seen {st[6]})",
        )


def build_globals_struct(
    Bar, instructions, timings,
    qkv_weights, attn_norm_weights, o_weights,
    expert_gate_weights, expert_up_weights, expert_down_weights, router_weights, ffn_ln_weights,
    lm_head_norm_weights, lm_head_weights,
    k_cache, v_cache, rope_cos, rope_sin,
    hidden_states, q_post_rope, attn_out, attn_lse_intermediates, attn_out_intermediates,
    expert_silu_out, router_normed_hidden, logits,
    selected_expert_indices, selected_expert_scores, predicted_expert_indices,
    pos_id, attn_scale, rms_norm_eps, skip_attn_reduction,
    *,
    expert_proj_block_size: int = 16,
    down_proj_block_size: int = 16,
    o_proj_block_size: int = 16,
    qkv_block_size: int = 16,
    attn_kv_block_size: int = 16,
    lm_head_block_size: int = 16,
    lm_head_reduction: int = 2048,
    router_bias=None,
    predictor_weights=None,
    status=None,
    spin_timeout_us: int = 0,
    record_timings: bool = False,
    work_sharing: bool = False,
    argmax_out=None,
    next_embed_weights=None,
    reset_for_next_launch: bool = False,
    downproj_overlap: bool = False,
    late_loads: bool = False,
) -> MkMixtralGlobals:
    """Validate the reference-ordered arguments and fill the C struct.

    Raises ``TypeError``/``ValueError`` for wrong dtypes, devices, layouts or
    inconsistent shapes, before anything reaches the GPU.
    """
    _check(isinstance(hidden_states, torch.Tensor), "hidden_states must be a torch.Tensor", TypeError)
    dev = hidden_states.device
    _check(dev.type == "cuda", f"mk_mixtral needs GPU tensors, hidden_states is on {dev}")
    bf16 = torch.bfloat16

    _check_tensor("expert_gate_weights", expert_gate_weights, bf16, dev)
    _check(expert_gate_weights.dim() == 3, "expert_gate_weights must be [L*E, F, H]")
    LE, F, H = expert_gate_weights.shape
    _check_tensor("ffn_ln_weights", ffn_ln_weights, bf16, dev)
    _check(ffn_ln_weights.dim() == 2 and ffn_ln_weights.shape[1] == H, "ffn_ln_weights must be [L, H]")
    L = ffn_ln_weights.shape[0]
    _check(L > 0 and LE % L == 0, f"expert depth {LE} is not a multiple of {L} layers")
    E = LE // L
    _check_tensor("expert_up_weights", expert_up_weights, bf16, dev, (LE, F, H))
    _check_tensor("expert_down_weights", expert_down_weights, bf16, dev, (LE, H, F))
    _check_tensor("router_weights", router_weights, bf16, dev, (LE, H))
    _check_tensor("hidden_states", hidden_states, bf16, dev, (H,))
    _check_tensor("expert_silu_out", expert_silu_out, bf16, dev, (E, F))
    _check_tensor("router_normed_hidden", router_normed_hidden, bf16, dev, (H,))
    _check_tensor("selected_expert_indices", selected_expert_indices, torch.int32, dev)
    k = selected_expert_indices.numel()
    _check_tensor("selected_expert_scores", selected_expert_scores, bf16, dev, (k,))
    _check_tensor("predicted_expert_indices", predicted_expert_indices, torch.int32, dev, (k,))
    _check(k == 2, f"num_experts_per_tok must be 2, got {k}")
    _check(2 <= E <= MAX_EXPERTS, f"num_experts must be in [2, {MAX_EXPERTS}], got {E}")
    _check(H % 512 == 0 and F % 512 == 0, f"hidden ({H}) and intermediate ({F}) sizes must be multiples of 512")

    _check_tensor("barriers", Bar, torch.int32, dev)
    _check(Bar.dim() == 3 and Bar.shape[0] >= L and Bar.shape[1] >= 8, "barriers must be [L, >=8, width]")
    _check_tensor("instructions", instructions, torch.int32, dev)
    _check(instructions.dim() == 3 and instructions.shape[2] == 32, "instructions must be [W, Q, 32]")
    W, Q, _ = instructions.shape
    _check(W > 0 and Q > 0, "empty instruction tensor")
    if timings is not None:
        _check_tensor("timings", timings, torch.int32, dev, (W, Q, 128))
    _check(record_timings is False or timings is not None, "record_timings needs a timings tensor")

    for name, bs, dim in (("expert_proj_block_size", expert_proj_block_size, F),
                          ("down_proj_block_size", down_proj_block_size, H),
                          ("o_proj_block_size", o_proj_block_size, H)):
        _check(int(bs) > 0 and dim % int(bs) == 0, f"{name}={bs} must divide {dim}")

    if router_bias is not None:
        _check_tensor("router_bias", router_bias, torch.float32, dev, min_numel=LE)
        _check(router_bias.numel() == LE, f"router_bias must have L*E={LE} elements")
    if predictor_weights is not None:
        _check_tensor("predictor_weights", predictor_weights, bf16, dev, (LE, H))
    if status is not None:
        _check_tensor("status", status, torch.int32, dev, min_numel=STATUS_WORDS)

    attn = _attention_shape(qkv_weights, attn_norm_weights, o_weights, lm_head_norm_weights, lm_head_weights,
                            k_cache, v_cache, rope_cos, rope_sin, q_post_rope, attn_out, attn_lse_intermediates,
                            attn_out_intermediates, logits, L, H, int(pos_id), dev, int(qkv_block_size),
                            int(attn_kv_block_size), int(lm_head_block_size), int(lm_head_reduction))

    g = MkMixtralGlobals()
    g.struct_size = ctypes.sizeof(MkMixtralGlobals)
    g.abi_version = ABI_VERSION
    g.barriers = Bar.data_ptr()
    g.bar_layers, g.bar_ops, g.bar_width = Bar.shape
    g.instructions = instructions.data_ptr()
    g.num_workers, g.queue_len = W, Q
    g.timings = None if timings is None else timings.data_ptr()
    for name, t in (("qkv_weights", qkv_weights), ("attn_norm_weights", attn_norm_weights),
                    ("o_weights", o_weights), ("lm_head_norm_weights", lm_head_norm_weights),
                    ("lm_head_weights", lm_head_weights), ("k_cache", k_cache), ("v_cache", v_cache),
                    ("rope_cos", rope_cos), ("rope_sin", rope_sin), ("q_post_rope", q_post_rope),
                    ("attn_out", attn_out), ("attn_lse_intermediates", attn_lse_intermediates),
                    ("attn_out_intermediates", attn_out_intermediates), ("logits", logits)):
        setattr(g, name, t.data_ptr() if isinstance(t, torch.Tensor) and t.numel() else None)
    g.expert_gate_weights = expert_gate_weights.data_ptr()
    g.expert_up_weights = expert_up_weights.data_ptr()
    g.expert_down_weights = expert_down_weights.data_ptr()
    g.router_weights = router_weights.data_ptr()
    g.ffn_ln_weights = ffn_ln_weights.data_ptr()
    g.hidden_states = hidden_states.data_ptr()
    g.expert_silu_out = expert_silu_out.data_ptr()
    g.router_normed_hidden = router_normed_hidden.data_ptr()
    g.selected_expert_indices = selected_expert_indices.data_ptr()
    g.selected_expert_scores = selected_expert_scores.data_ptr()
    g.predicted_expert_indices = predicted_expert_indices.data_ptr()
    g.pos_id = int(pos_id)
    g.attn_scale = float(attn_scale)
    g.rms_norm_eps = float(rms_norm_eps)
    g.skip_attn_reduction = int(bool(skip_attn_reduction))
    g.num_layers, g.hidden_size, g.intermediate_size = L, H, F
    g.num_experts, g.num_experts_per_tok = E, k
    g.expert_proj_block_size = int(expert_proj_block_size)
    g.down_proj_block_size = int(down_proj_block_size)
    g.o_proj_block_size = int(o_proj_block_size)
    if attn is not None:
        (g.qkv_block_size, g.attn_kv_block_size, g.lm_head_block_size, g.lm_head_reduction,
         g.num_attention_heads, g.num_kv_heads, g.head_dim, g.vocab_size, g.kv_capacity,
         g.attn_partial_slots) = attn
    else:
        for name in ("qkv_weights", "attn_norm_weights", "o_weights", "lm_head_norm_weights", "lm_head_weights",
                     "k_cache", "v_cache", "rope_cos", "rope_sin", "q_post_rope", "attn_out",
                     "attn_lse_intermediates", "attn_out_intermediates", "logits"):
            setattr(g, name, None)
    g.router_bias = None if router_bias is None else router_bias.data_ptr()
    g.predictor_weights = None if predictor_weights is None else predictor_weights.data_ptr()
    g.status = None if status is None else status.data_ptr()
    g.spin_timeout_us = int(spin_timeout_us)
    g.record_timings = int(bool(record_timings))
    g.work_sharing = int(bool(work_sharing))
    g.argmax_out, g.next_embed_weights = _decode_tail(argmax_out, next_embed_weights, attn is not None, dev, H)
    g.reset_for_next_launch = int(bool(reset_for_next_launch))
    g.downproj_overlap = int(bool(downproj_overlap))
    g.late_loads = int(bool(late_loads))
    return g


def _decode_tail(argmax_out, next_embed_weights, has_lm_head: bool, dev, H: int):
    """Pointers of the optional in-kernel argmax / next-token embedding."""
    if next_embed_weights is not None:
        _check(argmax_out is not None, "next_embed_weights needs argmax_out")
        _check_tensor("next_embed_weights", next_embed_weights, torch.bfloat16, dev)
        _check(next_embed_weights.dim() == 2 and next_embed_weights.shape[1] == H,
               f"next_embed_weights must be [V, {H}]")
    if argmax_out is None:
        return None, None
    _check(has_lm_head, "argmax_out needs the LM head (attention tensors)")
    _check(isinstance(argmax_out, torch.Tensor) and argmax_out.dtype == torch.int64 and argmax_out.device == dev
           and argmax_out.numel() >= 1, "argmax_out must be an int64 tensor on the launch device", TypeError)
    return argmax_out.data_ptr(), None if next_embed_weights is None else next_embed_weights.data_ptr()


def _attention_shape(qkv, attn_ln, o_proj, lm_norm, lm_head, k_cache, v_cache, rope_cos, rope_sin, q_rope,
                     attn_out, lse_int, out_int, logits, L, H, pos_id, dev, qkv_bs, kv_bs, lm_bs, lm_red):
    """Validate the attention-side tensors; None when they are absent (the
    MoE-only launch), else the struct's attention shape fields."""
    if not (isinstance(qkv, torch.Tensor) and qkv.numel()):
        return None
    bf16 = torch.bfloat16
    _check(k_cache.dim() == 4, "k_cache must be [L*B, T, Hkv, D] (batch 1)")
    LB, T, Hkv, D = k_cache.shape
    _check(LB == L, f"k_cache has {LB} layer rows, expected {L} (batch 1)")
    _check(D in (64, 128), f"head_dim must be 64 or 128, got {D}")
    _check_tensor("attn_lse_intermediates", lse_int, torch.float32, dev)
    _check(lse_int.dim() == 2, "attn_lse_intermediates must be [Hq, P]")
    Hq, P = lse_int.shape
    _check(Hkv > 0 and Hq % Hkv == 0 and 1 <= Hq // Hkv <= 4, f"need Hq / Hkv in 1..4, got {Hq} / {Hkv}")
    QKV = (Hq + 2 * Hkv) * D
    _check_tensor("qkv_weights", qkv, bf16, dev, (L, QKV, H))
    _check_tensor("attn_norm_weights", attn_ln, bf16, dev, (L, H))
    _check_tensor("o_weights", o_proj, bf16, dev, (L, H, Hq * D))
    _check_tensor("k_cache", k_cache, bf16, dev, (L, T, Hkv, D))
    _check_tensor("v_cache", v_cache, bf16, dev, (L, T, Hkv, D))
    _check_tensor("rope_cos", rope_cos, torch.float32, dev, min_numel=T * D)
    _check(rope_cos.dim() == 2 and rope_cos.shape[1] == D and rope_cos.shape[0] >= T, "rope_cos must be [T, D]")
    _check_tensor("rope_sin", rope_sin, torch.float32, dev, tuple(rope_cos.shape))
    _check_tensor("q_post_rope", q_rope, bf16, dev, (Hq * D,))
    _check_tensor("attn_out", attn_out, bf16, dev, (Hq * D,))
    _check_tensor("attn_out_intermediates", out_int, torch.float32, dev, (Hq, P, D))
    _check_tensor("logits", logits, bf16, dev)
    V = logits.numel()
    _check(logits.dim() == 1, "logits must be [V]")
    _check_tensor("lm_head_norm_weights", lm_norm, bf16, dev, min_numel=H)
    _check(lm_norm.numel() == H, "lm_head_norm_weights must have H elements")
    _check_tensor("lm_head_weights", lm_head, bf16, dev, (V, H))
    _check(0 <= pos_id < T, f"pos_id {pos_id} outside the KV cache ({T} positions)")
    _check(qkv_bs > 0 and D % qkv_bs == 0 and qkv_bs % 2 == 0, f"qkv_block_size {qkv_bs} must be even and divide {D}")
    _check(kv_bs > 0, "attn_kv_block_size must be positive")
    _check(lm_bs > 0 and lm_bs % 2 == 0 and V % lm_bs == 0, f"lm_head_block_size {lm_bs} must be even, divide {V}")
    _check(lm_red % 512 == 0 and lm_red > 0, "lm_head_reduction must be a multiple of 512")
    return qkv_bs, kv_bs, lm_bs, lm_red, Hq, Hkv, D, V, T, P


def launch_struct(g: MkMixtralGlobals, device: torch.device, stream=None) -> None:
    """Launch a pre-validated struct (the per-token fast path of the bench)."""
    lib = load_library()
    if stream is None:
        stream = torch.cuda.current_stream(device)
    rc = lib.mk_mixtral_launch(ctypes.byref(g), ctypes.c_void_p(stream.cuda_stream))
    if rc:
        raise MKError(rc, _error_text(lib, rc))


def mk_mixtral(*args, stream=None, debug_sync: bool = False, **kwargs):
    """Launch the persistent MoE megakernel; same positional arguments as the
    reference binding (``demos/mixtral/mixtral.cu:43-93``)."""
    if len(args) != 32:
        raise TypeError(f"mk_mixtral takes 32 positional arguments, got {len(args)}")
    load_library()
    g = build_globals_struct(*args, **kwargs)
    device = args[17].device
    with torch.cuda.device(device):
        launch_struct(g, device, stream)
        if debug_sync:
            raise_if_failed(device)
