"""``mk_llama`` -- the drop-in launcher module of the dense (Llama) VM.

The reference imports its compiled Llama kernel as a module from the build
directory (``megakernels/demos/latency/mk.py:50-63``) and calls it with 27
positional arguments in the field order of ``llama_3b_globals``
(``demos/low-latency-llama/llama_3b.cu:26-54``) plus ``stream=``.  This module
provides the same callable for the MI355X build: it validates the tensors,
fills the C-ABI struct of ``include/mk_llama.h`` and calls ``mk_llama_launch``
in ``libmk_mixtral.so`` (the library is shared with the Mixtral VM, and so
are its status words) through ctypes.  ``mk_llama_3b`` is the same callable
under the reference's 3B module name.

Keyword-only additions (defaults are the reference's compiled-in values):
the block sizes and ``matvec_reduction_size`` the instructions were built
with, ``spin_timeout_us``, ``record_timings``, ``argmax_out`` /
``next_embed_weights``, ``reset_for_next_launch``, ``late_loads`` (prefetch
off) and ``debug_sync`` (as in ``mk_mixtral``).  There is no fallback.
"""

from __future__ import annotations

import ctypes

import torch

import mk_mixtral
from mk_mixtral import MKError, _check, _check_tensor, _error_text, raise_if_failed

__all__ = ["mk_llama", "mk_llama_3b", "MkLlamaGlobals", "build_llama_struct"]

ABI_VERSION = 3
_P = ctypes.c_void_p


class MkLlamaGlobals(ctypes.Structure):
    """ctypes mirror of ``mk_llama_globals`` (include/mk_llama.h)."""

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
        ("mlp_norm_weights", _P),
        ("up_weights", _P),
        ("gate_weights", _P),
        ("down_weights", _P),
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
        ("silu_out", _P),
        ("logits", _P),
        ("pos_id", ctypes.c_uint32),
        ("attn_scale", ctypes.c_float),
        ("rms_norm_eps", ctypes.c_float),
        ("skip_attn_reduction", ctypes.c_int32),
        ("num_layers", ctypes.c_int32),
        ("hidden_size", ctypes.c_int32),
        ("intermediate_size", ctypes.c_int32),
        ("num_attention_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("vocab_size", ctypes.c_int32),
        ("kv_capacity", ctypes.c_int32),
        ("attn_partial_slots", ctypes.c_int32),
        ("up_gate_proj_block_size", ctypes.c_int32),
        ("down_proj_block_size", ctypes.c_int32),
        ("o_proj_block_size", ctypes.c_int32),
        ("qkv_block_size", ctypes.c_int32),
        ("attn_kv_block_size", ctypes.c_int32),
        ("lm_head_block_size", ctypes.c_int32),
        ("matvec_reduction_size", ctypes.c_int32),
        ("status", _P),
        ("spin_timeout_us", ctypes.c_uint32),
        ("record_timings", ctypes.c_int32),
        ("argmax_out", ctypes.c_void_p),
        ("next_embed_weights", ctypes.c_void_p),
        ("reset_for_next_launch", ctypes.c_int32),
        ("late_loads", ctypes.c_int32),
    ]


#: C entry points declared in include/mk_llama.h
EXPORTED_SYMBOLS = ("mk_llama_launch", "mk_llama_abi_version")

_bound = False


def load_library():
    """The shared library with the Llama entry points typed."""
    global _bound
    lib = mk_mixtral.load_library()
    if not _bound:
        lib.mk_llama_launch.argtypes = [ctypes.POINTER(MkLlamaGlobals), ctypes.c_void_p]
        lib.mk_llama_launch.restype = ctypes.c_int
        lib.mk_llama_abi_version.restype = ctypes.c_int
        if lib.mk_llama_abi_version() != ABI_VERSION:
            raise MKError(1, f"library has Llama ABI {lib.mk_llama_abi_version()}, expected {ABI_VERSION}")
        _bound = True
    return lib


def build_llama_struct(
    Bar, instructions, timings,
    qkv_weights, attn_norm_weights, o_weights, mlp_norm_weights, up_weights, gate_weights, down_weights,
    lm_head_norm_weights, lm_head_weights, k_cache, v_cache,
    rope_cos, rope_sin,
    hidden_states, q_post_rope, attn_out, attn_lse_intermediates, attn_out_intermediates, silu_out, logits,
    pos_id, attn_scale, rms_norm_eps, skip_attn_reduction,
    *,
    up_gate_proj_block_size: int = 16,
    down_proj_block_size: int = 16,
    o_proj_block_size: int = 16,
    qkv_block_size: int = 16,
    attn_kv_block_size: int = 16,
    lm_head_block_size: int = 16,
    matvec_reduction_size: int | None = None,
    status=None,
    spin_timeout_us: int = 0,
    record_timings: bool = False,
    argmax_out=None,
    next_embed_weights=None,
    reset_for_next_launch: bool = False,
    late_loads: bool = False,
) -> MkLlamaGlobals:
    """Validate the reference-ordered arguments and fill the C struct;
    ``TypeError``/``ValueError`` before anything reaches the GPU."""
    _check(isinstance(hidden_states, torch.Tensor), "hidden_states must be a torch.Tensor", TypeError)
    dev = hidden_states.device
    _check(dev.type == "cuda", f"mk_llama needs GPU tensors, hidden_states is on {dev}")
    bf16 = torch.bfloat16
    _check_tensor("up_weights", up_weights, bf16, dev)
    _check(up_weights.dim() == 3, "up_weights must be [L, F, H]")
    L, F, H = up_weights.shape
    _check_tensor("gate_weights", gate_weights, bf16, dev, (L, F, H))
    _check_tensor("down_weights", down_weights, bf16, dev, (L, H, F))
    _check_tensor("mlp_norm_weights", mlp_norm_weights, bf16, dev, (L, H))
    _check_tensor("attn_norm_weights", attn_norm_weights, bf16, dev, (L, H))
    _check_tensor("hidden_states", hidden_states, bf16, dev, (H,))
    _check_tensor("silu_out", silu_out, bf16, dev, (F,))
    _check(H % 512 == 0, f"hidden size {H} must be a multiple of 512")
    _check(k_cache.dim() == 4, "k_cache must be [L*B, T, Hkv, D] (batch 1)")
    _, T, Hkv, D = k_cache.shape
    _check(D in (64, 128), f"head_dim must be 64 or 128, got {D}")
    _check_tensor("attn_lse_intermediates", attn_lse_intermediates, torch.float32, dev)
    _check(attn_lse_intermediates.dim() == 2, "attn_lse_intermediates must be [Hq, P]")
    Hq, P = attn_lse_intermediates.shape
    _check(Hkv > 0 and Hq % Hkv == 0 and 1 <= Hq // Hkv <= 4, f"need Hq / Hkv in 1..4, got {Hq} / {Hkv}")
    _check((Hq * D) % 512 == 0, f"Hq * head_dim ({Hq * D}) must be a multiple of 512")
    _check_tensor("qkv_weights", qkv_weights, bf16, dev, (L, (Hq + 2 * Hkv) * D, H))
    _check_tensor("o_weights", o_weights, bf16, dev, (L, H, Hq * D))
    _check_tensor("k_cache", k_cache, bf16, dev, (L, T, Hkv, D))
    _check_tensor("v_cache", v_cache, bf16, dev, (L, T, Hkv, D))
    _check_tensor("rope_cos", rope_cos, torch.float32, dev)
    _check(rope_cos.dim() == 2 and rope_cos.shape[1] == D and rope_cos.shape[0] >= T, "rope_cos must be [>=T, D]")
    _check_tensor("rope_sin", rope_sin, torch.float32, dev, tuple(rope_cos.shape))
    _check_tensor("q_post_rope", q_post_rope, bf16, dev, (Hq * D,))
    _check_tensor("attn_out", attn_out, bf16, dev, (Hq * D,))
    _check_tensor("attn_out_intermediates", attn_out_intermediates, torch.float32, dev, (Hq, P, D))
    _check_tensor("logits", logits, bf16, dev)
    _check(logits.dim() == 1, "logits must be [V]")
    V = logits.numel()
    _check_tensor("lm_head_norm_weights", lm_head_norm_weights, bf16, dev)
    _check(lm_head_norm_weights.numel() == H, "lm_head_norm_weights must have H elements")
    _check_tensor("lm_head_weights", lm_head_weights, bf16, dev, (V, H))
    _check(0 <= int(pos_id) < T, f"pos_id {pos_id} outside the KV cache ({T} positions)")
    R = int(matvec_reduction_size) if matvec_reduction_size is not None else H
    _check(R % 512 == 0 and R > 0 and F % R == 0, f"matvec_reduction_size {R} must be a multiple of 512 dividing {F}")
    if R != F:
        _check(R // 512 in (1, 2, 4, 8), f"matvec_reduction_size {R} must be F ({F}) or 512, 1024, 2048, 4096")
        _check(int(down_proj_block_size) % (16 // (R // 512)) == 0,
               f"down_proj_block_size {down_proj_block_size} must be a multiple of {16 // (R // 512)} "
               f"(opcode-6 row group for matvec_reduction_size {R})")
    for name, bs, dim, even in (("up_gate_proj_block_size", up_gate_proj_block_size, F, False),
                                ("down_proj_block_size", down_proj_block_size, H, True),
                                ("o_proj_block_size", o_proj_block_size, H, True),
                                ("qkv_block_size", qkv_block_size, D, True),
                                ("lm_head_block_size", lm_head_block_size, V, True)):
        _check(int(bs) > 0 and dim % int(bs) == 0 and (not even or int(bs) % 2 == 0),
               f"{name}={bs} must {'be even and ' if even else ''}divide {dim}")
    _check(int(attn_kv_block_size) > 0, "attn_kv_block_size must be positive")
    _check_tensor("barriers", Bar, torch.int32, dev)
    _check(Bar.dim() == 3 and Bar.shape[0] >= L and Bar.shape[1] >= 7 and Bar.shape[2] >= Hq + 2 * Hkv,
           "barriers must be [L, >=7, >=Hq+2Hkv]")
    _check_tensor("instructions", instructions, torch.int32, dev)
    _check(instructions.dim() == 3 and instructions.shape[2] == 32, "instructions must be [W, Q, 32]")
    W, Q, _ = instructions.shape
    _check(W > 0 and Q > 0, "empty instruction tensor")
    if timings is not None:
        _check_tensor("timings", timings, torch.int32, dev, (W, Q, 128))
    _check(record_timings is False or timings is not None, "record_timings needs a timings tensor")
    if status is not None:
        _check_tensor("status", status, torch.int32, dev, min_numel=mk_mixtral.STATUS_WORDS)

    g = MkLlamaGlobals()
    g.struct_size = ctypes.sizeof(MkLlamaGlobals)
    g.abi_version = ABI_VERSION
    g.barriers = Bar.data_ptr()
    g.bar_layers, g.bar_ops, g.bar_width = Bar.shape
    g.instructions = instructions.data_ptr()
    g.num_workers, g.queue_len = W, Q
    g.timings = None if timings is None else timings.data_ptr()
    for name, t in (("qkv_weights", qkv_weights), ("attn_norm_weights", attn_norm_weights),
                    ("o_weights", o_weights), ("mlp_norm_weights", mlp_norm_weights), ("up_weights", up_weights),
                    ("gate_weights", gate_weights), ("down_weights", down_weights),
                    ("lm_head_norm_weights", lm_head_norm_weights), ("lm_head_weights", lm_head_weights),
                    ("k_cache", k_cache), ("v_cache", v_cache), ("rope_cos", rope_cos), ("rope_sin", rope_sin),
                    ("hidden_states", hidden_states), ("q_post_rope", q_post_rope), ("attn_out", attn_out),
                    ("attn_lse_intermediates", attn_lse_intermediates),
                    ("attn_out_intermediates", attn_out_intermediates), ("silu_out", silu_out),
                    ("logits", logits)):
        setattr(g, name, t.data_ptr())
    g.pos_id = int(pos_id)
    g.attn_scale = float(attn_scale)
    g.rms_norm_eps = float(rms_norm_eps)
    g.skip_attn_reduction = int(bool(skip_attn_reduction))
    g.num_layers, g.hidden_size, g.intermediate_size = L, H, F
    g.num_attention_heads, g.num_kv_heads, g.head_dim = Hq, Hkv, D
    g.vocab_size, g.kv_capacity, g.attn_partial_slots = V, T, P
    g.up_gate_proj_block_size = int(up_gate_proj_block_size)
    g.down_proj_block_size = int(down_proj_block_size)
    g.o_proj_block_size = int(o_proj_block_size)
    g.qkv_block_size = int(qkv_block_size)
    g.attn_kv_block_size = int(attn_kv_block_size)
    g.lm_head_block_size = int(lm_head_block_size)
    g.matvec_reduction_size = R
    g.status = None if status is None else status.data_ptr()
    g.spin_timeout_us = int(spin_timeout_us)
    g.record_timings = int(bool(record_timings))
    g.argmax_out, g.next_embed_weights = mk_mixtral._decode_tail(argmax_out, next_embed_weights, True, dev, H)
    g.reset_for_next_launch = int(bool(reset_for_next_launch))
    g.late_loads = int(bool(late_loads))
    return g


def launch_struct(g: MkLlamaGlobals, device: torch.device, stream=None) -> None:
    lib = load_library()
    if stream is None:
        stream = torch.cuda.current_stream(device)
    rc = lib.mk_llama_launch(ctypes.byref(g), ctypes.c_void_p(stream.cuda_stream))
    if rc:
        raise MKError(rc, _error_text(lib, rc))


def mk_llama(*args, stream=None, debug_sync: bool = False, **kwargs):
    """Launch one decode step of the dense VM; same positional arguments as
    the reference binding (``demos/low-latency-llama/llama_3b.cu:26-54``)."""
    if len(args) != 27:
        raise TypeError(f"mk_llama takes 27 positional arguments, got {len(args)}")
    load_library()
    g = build_llama_struct(*args, **kwargs)
    device = args[16].device
    with torch.cuda.device(device):
        launch_struct(g, device, stream)
        if debug_sync:
            raise_if_failed(device)


mk_llama_3b = mk_llama
