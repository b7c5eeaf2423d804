"""Synthetic looped language model: configs and seeded random-init weights.

The architecture follows the Huginn-style looped LM that the reference's
block forwards drive (src/decoding/huginn_blocks.py:1-30,
huginn_blocks_batch.py:1-31):

  P  x = wte(tok) * emb_scale -> n_prelude SandwichBlocks      (slots 0..n_prelude-1)
     e = x (static state, re-injected every recurrence); s0 = seeded trunc-normal
  R  s = adapter(cat[s, e]) -> n_core SandwichBlocks            (slot n_prelude + step*n_core + l)
     applied T_total times per token
  C  x = ln_f(s) -> n_coda SandwichBlocks -> ln_f -> lm_head    (slot n_prelude + T_total*n_core + i)

SandwichBlock: h = norm_1(x); q,k,v = split(h Wqkv^T); q,k = RoPE(q,k);
a = attn(q, slot prefix) Wproj^T; x = norm_2(a + x);
x = norm_4(mlp(norm_3(x)) + x), mlp(u) = (silu(u Wg^T) * (u Wu^T)) Wd^T.
RMSNorm everywhere, RoPE base 10000 on interleaved pairs, SwiGLU FFN, no biases.

Weights are drawn N(0, init_std) in float32 on the CPU from one
torch.Generator seeded with `seed`, in the fixed order of `param_specs`;
norm weights are 1. The same float32 tensors, rounded to the run dtype, feed
both the GPU model and the CPU oracle.
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np
import torch


@dataclass(frozen=True)
class LoopedLMConfig:
    name: str
    vocab_size: int
    d_model: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    n_prelude: int
    n_core: int
    n_coda: int
    T_total: int
    rope_base: float = 10000.0
    norm_eps: float = 1e-6
    emb_scale: float = 1.0
    init_std: float = 0.02
    state_std: float = 0.02
    dtype: str = "bfloat16"

    @property
    def torch_dtype(self) -> torch.dtype:
        return {"bfloat16": torch.bfloat16, "float32": torch.float32}[self.dtype]

    @property
    def qkv_dim(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim

    @property
    def n_slots(self) -> int:
        """Per-depth slot count: prelude + T_total * core + coda
        (src/decoding/kv_cache.py:12-15)."""
        return self.n_prelude + self.T_total * self.n_core + self.n_coda

    def with_(self, **kw) -> "LoopedLMConfig":
        return replace(self, **kw)


CONFIGS: dict[str, LoopedLMConfig] = {
    # tiny fp32 looped LM: d=256, 4 heads x 64, SwiGLU 1024, 1 + 2x4 + 1 layers, V=4096
    "tiny": LoopedLMConfig("tiny", 4096, 256, 4, 4, 64, 1024, 1, 2, 1, 4, dtype="float32"),
    # 2048-d bf16 looped LM: 16 heads x 128, SwiGLU 5632, 2 + 4x16 + 2 layers, V=32000
    "looped-2048": LoopedLMConfig("looped-2048", 32000, 2048, 16, 16, 128, 5632, 2, 4, 2, 16),
    # long-context GQA variant: 16 query / 4 kv heads x 128, 4-layer core looped 32 times
    "looped-2048-gqa": LoopedLMConfig("looped-2048-gqa", 32000, 2048, 16, 4, 128, 5632, 2, 4, 2, 32),
}


def param_specs(cfg: LoopedLMConfig) -> list[tuple[str, tuple[int, ...], str]]:
    """(name, shape, init) in generation order; init is 'normal' or 'ones'."""
    D, F = cfg.d_model, cfg.ffn
    specs: list[tuple[str, tuple[int, ...], str]] = [("wte", (cfg.vocab_size, D), "normal")]
    for part, count in (("prelude", cfg.n_prelude), ("core", cfg.n_core), ("coda", cfg.n_coda)):
        for i in range(count):
            p = f"{part}.{i}."
            specs += [
                (p + "Wqkv", (cfg.qkv_dim, D), "normal"),
                (p + "proj", (D, cfg.n_heads * cfg.head_dim), "normal"),
                (p + "fc", (2 * F, D), "normal"),
                (p + "mlp_proj", (D, F), "normal"),
                (p + "norm_1", (D,), "ones"),
                (p + "norm_2", (D,), "ones"),
                (p + "norm_3", (D,), "ones"),
                (p + "norm_4", (D,), "ones"),
            ]
    specs += [("adapter", (D, 2 * D), "normal"), ("ln_f", (D,), "ones"), ("lm_head", (cfg.vocab_size, D), "normal")]
    return specs


def init_weights(cfg: LoopedLMConfig, seed: int = 0) -> dict[str, torch.Tensor]:
    """float32 CPU weights, N(0, init_std) from one seeded generator, rounded
    through the run dtype (so the oracle sees exactly the GPU model's values)."""
    g = torch.Generator().manual_seed(seed)
    out: dict[str, torch.Tensor] = {}
    for name, shape, init in param_specs(cfg):
        if init == "ones":
            t = torch.ones(shape, dtype=torch.float32)
        else:
            t = torch.empty(shape, dtype=torch.float32).normal_(0.0, cfg.init_std, generator=g)
        out[name] = t.to(cfg.torch_dtype).to(torch.float32)
    return out


def weights_numpy(w: dict[str, torch.Tensor]) -> dict[str, np.ndarray]:
    return {k: v.numpy() for k, v in w.items()}


def rope_tables(max_pos: int, head_dim: int, base: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(max_pos, head_dim/2) float32 cos/sin of pos * base^(-2j/head_dim), computed in float64."""
    j = torch.arange(head_dim // 2, dtype=torch.float64)
    theta = base ** (-2.0 * j / head_dim)
    ang = torch.arange(max_pos, dtype=torch.float64)[:, None] * theta[None, :]
    return torch.cos(ang).to(torch.float32), torch.sin(ang).to(torch.float32)


def _trunc_normal_seeded(out32: torch.Tensor, seed: int, std: float) -> None:
    g = torch.Generator()
    g.manual_seed(seed & 0x7FFF_FFFF_FFFF)
    torch.nn.init.trunc_normal_(out32, mean=0.0, std=std, a=-3 * std, b=3 * std, generator=g)


def initial_state_tokens(cfg: LoopedLMConfig, positions, state_seed: int = 0, mode: str = "random") -> torch.Tensor:
    """(len(positions), D) float32 s0 draws, deterministic per (state_seed,
    position): trunc_normal(std, +-3 std; seed = state_seed*1_000_003 + p + 1) *
    emb_scale (src/decoding/parcae_blocks.py:129-146). mode 'zero' gives zeros."""
    out = torch.zeros(len(positions), cfg.d_model, dtype=torch.float32)
    if mode == "zero":
        return out
    for j, p in enumerate(positions):
        _trunc_normal_seeded(out[j], state_seed * 1_000_003 + int(p) + 1, cfg.state_std)
    return (out * cfg.emb_scale).to(cfg.torch_dtype).to(torch.float32)


def initial_state_prefill(cfg: LoopedLMConfig, length: int, state_seed: int = 0, mode: str = "random") -> torch.Tensor:
    """(length, D) float32 prompt s0: one stream seeded state_seed*1_000_003
    (src/decoding/parcae_blocks.py:148-156; shared by every sequence of a batch,
    huginn_blocks_batch.py:134-142)."""
    out = torch.zeros(1, length, cfg.d_model, dtype=torch.float32)
    if mode != "zero":
        _trunc_normal_seeded(out, state_seed * 1_000_003, cfg.state_std)
    return (out[0] * cfg.emb_scale).to(cfg.torch_dtype).to(torch.float32)
