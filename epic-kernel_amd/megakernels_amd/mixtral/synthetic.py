"""Random-init Mixtral-shaped weights for the benchmark configs.

No checkpoint is available offline, so every config runs on synthetic
weights: matrices N(0, std) in bf16 (std 0.02), RMSNorm weights ones (the
init of ``_RMSNorm`` at ``megakernels/mixtral/model.py:120-124``), residual
inputs N(0, 1).  The object returned by :func:`make_synthetic_mixtral` is
duck-typed like the reference's ``MixtralForCausalLM`` as far as
``make_globals`` needs (``.config``, ``.device``, ``.dtype``,
``.stacked_params``, ``.lm_head``, ``.stacked_kv_cache``, ``.model``), with
the stacked layout of ``megakernels/mixtral/model.py:486-565``: ``expert_gate``
= HF ``w1`` ``[L, E, F, H]``, ``expert_up`` = ``w3`` ``[L, E, F, H]``,
``expert_down`` = ``w2`` ``[L, E, H, F]``, ``router_weight`` ``[L, E, H]``.

Attention, LM-head and KV-cache tensors are empty placeholders: the MoE hot
path never reads them.
"""

from __future__ import annotations

from dataclasses import dataclass, replace
from types import SimpleNamespace
from typing import Optional

import torch


@dataclass(frozen=True)
class MoEConfig:
    num_hidden_layers: int
    hidden_size: int
    intermediate_size: int
    num_attention_heads: int
    num_key_value_heads: int
    num_local_experts: int
    num_experts_per_tok: int
    vocab_size: int
    rms_norm_eps: float = 1e-5
    rope_theta: float = 1e6

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


#: BASELINE config 1: small MoE decode layer (plumbing; MALL-resident)
C1 = MoEConfig(1, 1024, 3584, 8, 2, 8, 2, 32000)
#: BASELINE config 2: one full-size Mixtral-8x7B MoE layer
C2 = MoEConfig(1, 4096, 14336, 32, 8, 8, 2, 32000)
#: the reference's small debug shapes (demos/mixtral/debug_mixtral_mk.py:38-48)
SMALL = MoEConfig(1, 512, 1024, 8, 2, 4, 2, 256)

#: BASELINE configs 4 and 5: the full Mixtral-8x7B shape (32 layers, 32 query
#: / 8 KV heads, head dim 128, vocab 32000, RoPE theta 1e6); they differ in the
#: pre-filled context (4096 vs 16384 positions), set by the decode driver
C4 = MoEConfig(32, 4096, 14336, 32, 8, 8, 2, 32000)
#: the smallest shape with an LM head: the reference splits the LM head's
#: reduction into 2048-column blocks (megakernels/mixtral/scheduler.py:236)
TINY = MoEConfig(2, 2048, 1024, 16, 4, 4, 2, 512)

CONFIGS = {"c1": C1, "c2": C2, "small": SMALL, "c4": C4, "tiny": TINY}


@dataclass
class StackedMoEParams:
    qkv_proj: torch.Tensor
    attn_ln_weight: torch.Tensor
    o_proj: torch.Tensor
    ffn_ln_weight: torch.Tensor
    router_weight: torch.Tensor
    expert_gate: torch.Tensor
    expert_up: torch.Tensor
    expert_down: torch.Tensor
    router_bias: Optional[torch.Tensor] = None
    predictor_weight: Optional[torch.Tensor] = None


def rope_tables(positions: int, head_dim: int, theta: float, device="cpu"):
    """RoPE cos/sin ``[positions, head_dim]`` fp32 in the interleaved layout
    the reference's kernels and python_vm use (``megakernels/mixtral/
    model.py:251-277``: Llama RoPE, columns permuted so that the pair
    (2i, 2i+1) shares frequency i): ``cos[p, 2i] = cos[p, 2i+1] = cos(p *
    theta^(-2i/D))``, likewise ``sin``."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim))
    ang = torch.arange(positions, dtype=torch.float64)[:, None] * inv_freq[None, :]
    cos = torch.repeat_interleave(torch.cos(ang), 2, dim=1).to(torch.float32)
    sin = torch.repeat_interleave(torch.sin(ang), 2, dim=1).to(torch.float32)
    return cos.to(device), sin.to(device)


def _normal(shape, std, gen, device, dtype=torch.bfloat16):
    return torch.empty(shape, dtype=dtype, device=device).normal_(0.0, std, generator=gen)


def make_synthetic_mixtral(
    config: MoEConfig,
    device="cpu",
    seed: int = 0,
    std: float = 0.02,
    ln_weight_std: float | None = None,
    router_bias: Optional[list[float]] = None,
    predictor_sigma: float | None = None,
    full: bool = False,
    kv_positions: int = 0,
    prefill: int = 0,
):
    """Build stacked random weights for ``config`` on ``device``.

    ``full=True`` adds what whole-model decode needs: QKV and O projections,
    attention RMSNorm, LM head and its norm, token embeddings N(0, 1), RoPE
    tables, and a KV cache ``[L, 1, kv_positions, Hkv, D]`` whose first
    ``prefill`` positions hold N(0, 1).  These are drawn from a second
    generator (seed + 1000003), so the MoE weights and the residual stream
    are the same with or without them.

    ``ln_weight_std`` draws the FFN RMSNorm weights as ``1 + N(0, s)`` instead
    of ones (exercises the norm-weight rounding step in tests).
    ``router_bias`` (per-expert list) and ``predictor_sigma`` (noise std on a
    predictor copy of the router) enable the two optional extensions.
    """
    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    L, H, F, E = (config.num_hidden_layers, config.hidden_size,
                  config.intermediate_size, config.num_local_experts)
    dt = torch.bfloat16
    router = _normal([L, E, H], std, gen, device)
    gate = _normal([L, E, F, H], std, gen, device)
    up = _normal([L, E, F, H], std, gen, device)
    down = _normal([L, E, H, F], std, gen, device)
    if ln_weight_std is None:
        ffn_ln = torch.ones([L, H], dtype=dt, device=device)
    else:
        ffn_ln = (1.0 + _normal([L, H], ln_weight_std, gen, device, torch.float32)).to(dt)
    bias = None
    if router_bias is not None:
        bias = torch.tensor(router_bias, dtype=torch.float32, device=device).expand(L, E).contiguous()
    predictor = None
    if predictor_sigma is not None:
        predictor = (router.float() + _normal([L, E, H], predictor_sigma, gen, device, torch.float32)).to(dt)
    empty = torch.empty(0, dtype=dt, device=device)
    qkv = o_proj = attn_ln = lm_w = embed = empty
    lm_norm = torch.ones(H, dtype=dt, device=device)
    k_cache = v_cache = empty
    cos = sin = torch.empty(0, device=device)
    if full:
        g2 = torch.Generator(device=device)
        g2.manual_seed(seed + 1000003)
        Hq, Hkv, D, V = config.num_attention_heads, config.num_key_value_heads, config.head_dim, config.vocab_size
        qkv = _normal([L, (Hq + 2 * Hkv) * D, H], std, g2, device)
        o_proj = _normal([L, H, Hq * D], std, g2, device)
        if ln_weight_std is None:
            attn_ln = torch.ones([L, H], dtype=dt, device=device)
        else:
            attn_ln = (1.0 + _normal([L, H], ln_weight_std, g2, device, torch.float32)).to(dt)
        lm_w = _normal([V, H], std, g2, device)
        embed = _normal([V, H], 1.0, g2, device)
        T = max(kv_positions, prefill + 1)
        k_cache = torch.zeros([L, 1, T, Hkv, D], dtype=dt, device=device)
        v_cache = torch.zeros([L, 1, T, Hkv, D], dtype=dt, device=device)
        if prefill:
            k_cache[:, :, :prefill] = _normal([L, 1, prefill, Hkv, D], 1.0, g2, device)
            v_cache[:, :, :prefill] = _normal([L, 1, prefill, Hkv, D], 1.0, g2, device)
        cos, sin = rope_tables(T, D, config.rope_theta, device)
    params = StackedMoEParams(
        qkv_proj=qkv, attn_ln_weight=attn_ln, o_proj=o_proj, ffn_ln_weight=ffn_ln,
        router_weight=router, expert_gate=gate, expert_up=up, expert_down=down,
        router_bias=bias, predictor_weight=predictor,
    )
    return SimpleNamespace(
        config=config,
        device=device,
        dtype=dt,
        stacked_params=params,
        lm_head=SimpleNamespace(input_norm=SimpleNamespace(weight=lm_norm),
                                lm_head=SimpleNamespace(weight=lm_w)),
        embed_tokens=embed,
        stacked_kv_cache=(k_cache, v_cache),
        model=SimpleNamespace(rope_cos=cos, rope_sin=sin),
        # the seeded stream continues here: residual inputs are drawn after
        # the weights, so they are independent of every weight row
        generator=gen,
    )


def make_residuals(n_tokens: int, hidden: int, generator: torch.Generator | None = None, seed: int = 0,
                   device=None) -> torch.Tensor:
    """``n_tokens`` residual inputs N(0, 1) in bf16, ``[n, H]``, drawn from
    ``generator`` (normally ``model.generator``, continuing the weight stream)
    or, without one, from a fresh generator seeded ``seed``."""
    if generator is None:
        generator = torch.Generator(device=torch.device(device or "cpu"))
        generator.manual_seed(seed)
    dev = generator.device
    return torch.empty([n_tokens, hidden], dtype=torch.bfloat16, device=dev).normal_(0.0, 1.0, generator=generator)


def with_layers(config: MoEConfig, layers: int) -> MoEConfig:
    return replace(config, num_hidden_layers=layers)


def to_device(model, device):
    """Copy of a synthetic model with every tensor moved to ``device``."""
    device = torch.device(device)

    def mv(t):
        return None if t is None else t.to(device)

    sp = model.stacked_params
    params = StackedMoEParams(**{k: mv(v) for k, v in vars(sp).items()})
    return SimpleNamespace(
        config=model.config,
        device=device,
        dtype=model.dtype,
        stacked_params=params,
        lm_head=SimpleNamespace(input_norm=SimpleNamespace(weight=mv(model.lm_head.input_norm.weight)),
                                lm_head=SimpleNamespace(weight=mv(model.lm_head.lm_head.weight))),
        embed_tokens=mv(getattr(model, "embed_tokens", None)),
        stacked_kv_cache=tuple(mv(t) for t in model.stacked_kv_cache),
        model=SimpleNamespace(rope_cos=mv(model.model.rope_cos), rope_sin=mv(model.model.rope_sin)),
        generator=None,
    )


def slice_layers(model, layers: int, device="cpu"):
    """The first ``layers`` layers of a synthetic model (stacked weights and
    KV cache), with its embeddings, LM head and RoPE tables, copied to
    ``device``: a whole-model schedule over the slice runs the same
    per-layer work at the same shapes."""
    device = torch.device(device)

    def mv(t, cut=True):
        if t is None:
            return None
        t = t[:layers] if cut and t.dim() > 0 and t.shape[0] == model.config.num_hidden_layers else t
        return t.to(device).contiguous()

    sp = model.stacked_params
    params = StackedMoEParams(**{k: mv(v) for k, v in vars(sp).items()})
    return SimpleNamespace(
        config=with_layers(model.config, layers),
        device=device,
        dtype=model.dtype,
        stacked_params=params,
        lm_head=SimpleNamespace(input_norm=SimpleNamespace(weight=mv(model.lm_head.input_norm.weight, False)),
                                lm_head=SimpleNamespace(weight=mv(model.lm_head.lm_head.weight, False))),
        embed_tokens=mv(getattr(model, "embed_tokens", None), False),
        stacked_kv_cache=tuple(mv(t) for t in model.stacked_kv_cache),
        model=SimpleNamespace(rope_cos=mv(model.model.rope_cos, False), rope_sin=mv(model.model.rope_sin, False)),
        generator=None,
    )
