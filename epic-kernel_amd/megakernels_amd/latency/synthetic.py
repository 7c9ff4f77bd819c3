"""Random-init Llama-shaped weights for the dense decode config.

No checkpoint is available offline, so the dense VM runs on synthetic
weights: matrices N(0, std) in bf16 (std 0.02), RMSNorm weights ones (or
``1 + N(0, s)`` for tests), token embeddings and the pre-filled KV cache
N(0, 1).  The returned object is duck-typed like the reference's
``LlamaForCausalLM`` as far as ``make_globals`` needs (``.config``,
``.device``, ``.dtype``, ``.stacked_params``, ``.lm_head``,
``.stacked_kv_cache``, ``.model.rope_cos/rope_sin``), with the stacked layout
of ``megakernels/llama.py:491-499, 713-760``: ``qkv_proj`` ``[L, (Hq+2Hkv)D,
H]``, ``o_proj`` ``[L, H, Hq D]``, ``up_proj``/``gate_proj`` ``[L, F, H]``,
``down_proj`` ``[L, H, F]``, KV cache ``[L, 1, T, Hkv, D]``.

RoPE tables are the interleaved layout of ``megakernels/llama.py:452-470``
with plain ``theta^(-2i/D)`` frequencies (the Llama-3 frequency rescaling of
a real checkpoint's config does not apply to random-init weights).
"""

from __future__ import annotations

from dataclasses import dataclass, replace
from types import SimpleNamespace

import torch

from ..mixtral.synthetic import _normal, rope_tables


@dataclass(frozen=True)
class LlamaConfig:
    num_hidden_layers: int
    hidden_size: int
    intermediate_size: int
    num_attention_heads: int
    num_key_value_heads: int
    vocab_size: int
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


#: BASELINE config 3: Llama-3.2-3B shape (28 layers, hidden 3072, 24 query /
#: 8 KV heads, head dim 128, FFN 8192, vocab 128256, RoPE theta 500000)
C3 = LlamaConfig(28, 3072, 8192, 24, 8, 128256)
#: small shapes for parity tests: GQA 3 with head dim 128 and four down-
#: projection column chunks (gcd(2048, 1536) = 512), and GQA 4 with head dim 64
LLAMA_SMALL = LlamaConfig(2, 1536, 2048, 12, 4, 512)
LLAMA_TINY = LlamaConfig(2, 1024, 1536, 16, 4, 256)

CONFIGS = {"c3": C3, "small": LLAMA_SMALL, "tiny": LLAMA_TINY}


@dataclass
class StackedParams:
    qkv_proj: torch.Tensor
    o_proj: torch.Tensor
    attn_ln_weight: torch.Tensor
    mlp_ln_weight: torch.Tensor
    up_proj: torch.Tensor
    gate_proj: torch.Tensor
    down_proj: torch.Tensor


def make_synthetic_llama(config: LlamaConfig, device="cpu", seed: int = 0, std: float = 0.02,
                         ln_weight_std: float | None = None, kv_positions: int = 0, prefill: int = 0):
    """Stacked random weights for ``config`` on ``device``; the KV cache holds
    ``max(kv_positions, prefill + 1)`` positions, the first ``prefill`` of
    them N(0, 1)."""
    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    c = config
    L, H, F = c.num_hidden_layers, c.hidden_size, c.intermediate_size
    Hq, Hkv, D, V = c.num_attention_heads, c.num_key_value_heads, c.head_dim, c.vocab_size
    dt = torch.bfloat16

    def norm_w(shape):
        if ln_weight_std is None:
            return torch.ones(shape, dtype=dt, device=device)
        return (1.0 + _normal(shape, ln_weight_std, gen, device, torch.float32)).to(dt)

    params = StackedParams(
        qkv_proj=_normal([L, (Hq + 2 * Hkv) * D, H], std, gen, device),
        o_proj=_normal([L, H, Hq * D], std, gen, device),
        attn_ln_weight=norm_w([L, H]),
        mlp_ln_weight=norm_w([L, H]),
        up_proj=_normal([L, F, H], std, gen, device),
        gate_proj=_normal([L, F, H], std, gen, device),
        down_proj=_normal([L, H, F], std, gen, device),
    )
    lm_norm = norm_w([H])
    lm_w = _normal([V, H], std, gen, device)
    embed = _normal([V, H], 1.0, gen, device)
    T = max(kv_positions, prefill + 1)
    k_cache = torch.zeros([L, 1, T, Hkv, D], dtype=dt, device=device)
    v_cache = torch.zeros([L, 1, T, Hkv, D], dtype=dt, device=device)
    if prefill:
        k_cache[:, :, :prefill] = _normal([L, 1, prefill, Hkv, D], 1.0, gen, device)
        v_cache[:, :, :prefill] = _normal([L, 1, prefill, Hkv, D], 1.0, gen, device)
    cos, sin = rope_tables(T, D, c.rope_theta, device)
    return SimpleNamespace(
        config=c,
        device=device,
        dtype=dt,
        stacked_params=params,
        lm_head=SimpleNamespace(input_norm=SimpleNamespace(weight=lm_norm), lm_head=SimpleNamespace(weight=lm_w)),
        embed_tokens=embed,
        stacked_kv_cache=(k_cache, v_cache),
        model=SimpleNamespace(rope_cos=cos, rope_sin=sin),
    )


def with_layers(config: LlamaConfig, layers: int) -> LlamaConfig:
    return replace(config, num_hidden_layers=layers)


def to_device(model, device):
    """Copy of a synthetic Llama with every tensor moved to ``device``."""
    device = torch.device(device)
    sp = model.stacked_params
    return SimpleNamespace(
        config=model.config,
        device=device,
        dtype=model.dtype,
        stacked_params=StackedParams(**{k: v.to(device) for k, v in vars(sp).items()}),
        lm_head=SimpleNamespace(input_norm=SimpleNamespace(weight=model.lm_head.input_norm.weight.to(device)),
                                lm_head=SimpleNamespace(weight=model.lm_head.lm_head.weight.to(device))),
        embed_tokens=model.embed_tokens.to(device),
        stacked_kv_cache=tuple(t.to(device) for t in model.stacked_kv_cache),
        model=SimpleNamespace(rope_cos=model.model.rope_cos.to(device), rope_sin=model.model.rope_sin.to(device)),
    )
