"""Pins of the oracle's composed P / R / C forward (CPU).

The per-op pieces of the oracle are pinned in test_oracle_kernels.py. This
file pins how they are wired together -- the SandwichBlock of the
reference's single-token block (src/decoding/huginn_blocks.py:93-103:
h = norm_1(x); q, k, v = Wqkv h + RoPE; att = proj(attn); x = norm_2(att + x);
x = norm_4(mlp(norm_3(x)) + x)), the adapter on cat[s, e] (:216), the coda's
ln_f -> coda blocks -> ln_f -> lm_head (:261-292) and the per-depth slots
(src/decoding/kv_cache.py:12-15) -- by checks that fix the result
independently of the oracle's own code:

* closed forms: Wqkv = 0 and fc = 0 reduce a block to
  norm_4(norm_2(x)); a lone key (position 0) makes attention return that
  key's value, so the block is a fixed chain on one row;
* the adapter's halves: with adapter = [I | 0] the loop step reads s alone,
  with [0 | I] it reads e alone;
* a dense, whole-sequence formulation in torch (library RMSNorm, linear,
  SiLU, complex-multiplication RoPE, and causal scaled_dot_product_attention
  over all prompt positions at once, one pass per (loop step, layer)) must
  give the per-token, per-slot oracle's logits and slot caches.

Every norm weight is drawn away from 1 so that swapped norms show. The
mutation tests at the bottom plant wiring slips in the oracle and check that
these pins catch each one.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import kernels as K
from oracle.looped_lm import OracleLM


@dataclass(frozen=True)
class Cfg:
    vocab_size: int = 50
    d_model: int = 64
    n_heads: int = 4
    n_kv_heads: int = 2
    head_dim: int = 16
    ffn: int = 96
    n_prelude: int = 1
    n_core: int = 2
    n_coda: int = 1
    T_total: int = 3
    rope_base: float = 10000.0
    norm_eps: float = 1e-6
    emb_scale: float = 1.5


CFG = Cfg()


def _weights(cfg: Cfg, seed: int = 0) -> dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    D, F_ = cfg.d_model, cfg.ffn
    qkv = (cfg.n_heads + 2 * cfg.n_kv_heads) * cfg.head_dim
    w = {"wte": rng.normal(0, 0.5, (cfg.vocab_size, D)), "adapter": rng.normal(0, 0.15, (D, 2 * D)),
         "ln_f": 1 + 0.3 * rng.normal(size=D), "lm_head": rng.normal(0, 0.2, (cfg.vocab_size, D))}
    for part, count in (("prelude", cfg.n_prelude), ("core", cfg.n_core), ("coda", cfg.n_coda)):
        for i in range(count):
            p = f"{part}.{i}."
            w[p + "Wqkv"] = rng.normal(0, 0.2, (qkv, D))
            w[p + "proj"] = rng.normal(0, 0.2, (D, cfg.n_heads * cfg.head_dim))
            w[p + "fc"] = rng.normal(0, 0.2, (2 * F_, D))
            w[p + "mlp_proj"] = rng.normal(0, 0.15, (D, F_))
            for j in (1, 2, 3, 4):
                w[p + f"norm_{j}"] = 1 + 0.3 * rng.normal(size=D)
    return {k: v.astype(np.float32) for k, v in w.items()}


def _s0(L: int, D: int, seed: int = 5) -> np.ndarray:
    return np.random.default_rng(seed).normal(0, 0.3, (L, D)).astype(np.float32)


def _lm(w, cls=OracleLM, L: int = 16):
    return cls(CFG, w, L, 1, s0_tokens=lambda p: _s0(L, CFG.d_model)[p], s0_prefill=lambda n: _s0(L, CFG.d_model)[:n])


def _rms(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """RMSNorm through the library routine (float64)."""
    t = torch.from_numpy(np.asarray(x, dtype=np.float64))
    return (F.rms_norm(t, (t.shape[-1],), eps=CFG.norm_eps) * torch.from_numpy(w.astype(np.float64))).numpy()


def _close(a, b, tol=2e-5) -> bool:
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)) <= tol


# ---------------------------------------------------------------------------
# the pins, as predicates (the mutation tests reuse them)
# ---------------------------------------------------------------------------
def pin_zero_attention_and_mlp(cls=OracleLM) -> bool:
    """Wqkv = 0: q = k = v = 0, so attention returns 0 and proj adds nothing;
    fc = 0: the gated MLP returns 0. The block is then exactly
    norm_4(norm_2(x)) -- the residual enters each norm, norms in sandwich order."""
    w = _weights(CFG, 1)
    for i in range(CFG.n_core):
        w[f"core.{i}.Wqkv"][:] = 0
        w[f"core.{i}.fc"][:] = 0
    lm = _lm(w, cls)
    x = np.random.default_rng(2).normal(0, 1, CFG.d_model).astype(np.float32)
    got = lm.block("core.0.", x, slot=lm.slot_core(0, 0), b=0, pos=3)
    want = _rms(_rms(x, w["core.0.norm_2"]), w["core.0.norm_4"])
    return _close(got, want)


def pin_single_key_block(cls=OracleLM) -> bool:
    """At position 0 a query sees one key, its own: attention returns that
    position's value vector (per kv head; GQA head h reads kv head h // G) and
    RoPE at angle 0 is the identity. The block is then a fixed chain of
    library calls on one row (huginn_blocks.py:93-103)."""
    w = _weights(CFG, 3)
    lm = _lm(w, cls)
    x = np.random.default_rng(4).normal(0, 1, CFG.d_model).astype(np.float32)
    got = lm.block("core.1.", x, slot=lm.slot_core(2, 1), b=0, pos=0)
    p = "core.1."
    H, Hkv, Dh = CFG.n_heads, CFG.n_kv_heads, CFG.head_dim
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    xt = t(x)
    h = F.rms_norm(xt, (CFG.d_model,), eps=CFG.norm_eps) * t(w[p + "norm_1"])
    qkv = F.linear(h, t(w[p + "Wqkv"]))
    v = qkv[(H + Hkv) * Dh:].view(Hkv, Dh)
    o = v.repeat_interleave(H // Hkv, dim=0).reshape(-1)
    x1 = F.rms_norm(F.linear(o, t(w[p + "proj"])) + xt, (CFG.d_model,), eps=CFG.norm_eps) * t(w[p + "norm_2"])
    gu = F.linear(F.rms_norm(x1, (CFG.d_model,), eps=CFG.norm_eps) * t(w[p + "norm_3"]), t(w[p + "fc"]))
    m = F.linear(F.silu(gu[: CFG.ffn]) * gu[CFG.ffn:], t(w[p + "mlp_proj"]))
    want = F.rms_norm(m + x1, (CFG.d_model,), eps=CFG.norm_eps) * t(w[p + "norm_4"])
    return _close(got, want.numpy())


def pin_adapter_halves(cls=OracleLM) -> bool:
    """adapter = [I | 0] -> the loop step's input is s; [0 | I] -> it is e
    (the adapter acts on cat[s, e], huginn_blocks.py:216): a core call must
    then ignore the other half entirely."""
    D = CFG.d_model
    rng = np.random.default_rng(6)
    s, e, e2, s2 = (rng.normal(0, 1, D).astype(np.float32) for _ in range(4))
    ok = True
    for left, reads_s in ((np.eye(D), True), (np.zeros((D, D)), False)):
        w = _weights(CFG, 7)
        w["adapter"] = np.concatenate([left, np.eye(D) - left], axis=1).astype(np.float32)
        outs = []
        for ss, ee in ((s, e), (s, e2) if reads_s else (s2, e)):
            lm = _lm(w, cls)
            outs.append(lm.core(0, 2, 1, ss, ee))
        ok &= np.array_equal(outs[0], outs[1])
    return ok


def _dense_forward(w, ids, s0):
    """Whole prompt at once, in float64 torch: every (loop step, layer) pass
    runs causal SDPA over all positions (the per-slot cache of that pass is
    exactly the keys of earlier positions at the same step and layer).
    Returns (logits (L, V), {slot: (k (L, Hkv, Dh), v)})."""
    c = CFG
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    L = len(ids)
    H, Hkv, Dh = c.n_heads, c.n_kv_heads, c.head_dim
    j = torch.arange(Dh // 2, dtype=torch.float64)
    ang = torch.arange(L, dtype=torch.float64)[:, None] * (c.rope_base ** (-2.0 * j / Dh))[None, :]
    rot = torch.polar(torch.ones_like(ang), ang)  # e^{i pos theta_j}, (L, Dh/2)

    def rope(x):  # (L, heads, Dh): interleaved pairs as complex numbers
        z = torch.view_as_complex(x.reshape(L, x.shape[1], Dh // 2, 2).contiguous())
        return torch.view_as_real(z * rot[:, None, :]).reshape(L, x.shape[1], Dh)

    def norm(x, name):
        return F.rms_norm(x, (c.d_model,), eps=c.norm_eps) * t(w[name])

    caches = {}

    def block(p, x, slot):
        qkv = F.linear(norm(x, p + "norm_1"), t(w[p + "Wqkv"]))
        q = rope(qkv[:, : H * Dh].view(L, H, Dh))
        k = rope(qkv[:, H * Dh: (H + Hkv) * Dh].view(L, Hkv, Dh))
        v = qkv[:, (H + Hkv) * Dh:].view(L, Hkv, Dh)
        caches[slot] = (k.numpy(), v.numpy())
        rep = lambda a: a.repeat_interleave(H // Hkv, dim=1).transpose(0, 1)  # noqa: E731  (H, L, Dh)
        o = F.scaled_dot_product_attention(q.transpose(0, 1), rep(k), rep(v), is_causal=True)
        x = norm(F.linear(o.transpose(0, 1).reshape(L, H * Dh), t(w[p + "proj"])) + x, p + "norm_2")
        gu = F.linear(norm(x, p + "norm_3"), t(w[p + "fc"]))
        m = F.linear(F.silu(gu[:, : c.ffn]) * gu[:, c.ffn:], t(w[p + "mlp_proj"]))
        return norm(m + x, p + "norm_4")

    x = t(w["wte"])[torch.as_tensor(ids)] * c.emb_scale
    for i in range(c.n_prelude):
        x = block(f"prelude.{i}.", x, i)
    e, s = x, t(s0)
    for r in range(c.T_total):
        x = F.linear(torch.cat([s, e], dim=1), t(w["adapter"]))
        for l in range(c.n_core):
            x = block(f"core.{l}.", x, c.n_prelude + r * c.n_core + l)
        s = x
    x = norm(s, "ln_f")
    for i in range(c.n_coda):
        x = block(f"coda.{i}.", x, c.n_prelude + c.T_total * c.n_core + i)
    return F.linear(norm(x, "ln_f"), t(w["lm_head"])).numpy(), caches


def pin_dense_causal_prefill(cls=OracleLM) -> bool:
    """The per-token, per-slot oracle prefill (one position at a time through
    the full depth) equals the dense causal formulation: last-position logits
    and every slot cache's rows."""
    w = _weights(CFG, 8)
    ids = [3, 17, 42, 8, 8, 29, 0, 11]
    L = len(ids)
    lm = _lm(w, cls)
    got = lm.prefill(0, ids)
    want, caches = _dense_forward(w, ids, _s0(16, CFG.d_model)[:L])
    ok = _close(got, want[-1], 1e-4)
    for slot, (k, v) in caches.items():
        ok &= _close(lm.Kc[slot, 0, :L], k, 1e-4) and _close(lm.Vc[slot, 0, :L], v, 1e-4)
    return ok


PINS = [pin_zero_attention_and_mlp, pin_single_key_block, pin_adapter_halves, pin_dense_causal_prefill]


@pytest.mark.parametrize("pin", PINS, ids=lambda f: f.__name__)
def test_oracle_composition(pin):
    assert pin()


# ---------------------------------------------------------------------------
# mutation tests: wiring slips planted in the oracle must fail a pin
# ---------------------------------------------------------------------------
def _mutant_block(kind):
    def block(self, prefix, x, slot, b, pos):
        c, w = self.c, self.w
        H, Hkv, Dh = c.n_heads, c.n_kv_heads, c.head_dim
        h = K.rmsnorm(x, w[prefix + "norm_1"], c.norm_eps)
        qkv = K.linear_row(h, w[prefix + "Wqkv"])
        q = K.rope(qkv[: H * Dh].reshape(H, Dh), pos, self.cos, self.sin)
        k = K.rope(qkv[H * Dh: (H + Hkv) * Dh].reshape(Hkv, Dh), pos, self.cos, self.sin)
        v = qkv[(H + Hkv) * Dh:].reshape(Hkv, Dh)
        self.Kc[slot, b, pos] = k
        self.Vc[slot, b, pos] = v
        o = K.attention(q, self.Kc[slot, b], self.Vc[slot, b], pos + 1)
        a = K.linear_row(o.reshape(-1), w[prefix + "proj"])
        n2, n3 = ("norm_3", "norm_2") if kind == "swap_norm23" else ("norm_2", "norm_3")
        if kind == "residual_after_norm":
            x = K.rmsnorm(a, w[prefix + n2], c.norm_eps) + x
        else:
            x = K.rmsnorm(a + x, w[prefix + n2], c.norm_eps)
        gu = K.linear_row(K.rmsnorm(x, w[prefix + n3], c.norm_eps), w[prefix + "fc"])
        if kind == "swap_gate_up":
            gu = np.concatenate([gu[c.ffn:], gu[: c.ffn]])
        m = K.linear_row(K.swiglu(gu[: c.ffn], gu[c.ffn:]), w[prefix + "mlp_proj"])
        if kind == "mlp_residual_from_block_input":
            return K.rmsnorm(m + h, w[prefix + "norm_4"], c.norm_eps)
        return K.rmsnorm(m + x, w[prefix + "norm_4"], c.norm_eps)

    return type(f"Mutant_{kind}", (OracleLM,), {"block": block})


class SwappedAdapterHalves(OracleLM):
    def core(self, b, pos, step, s, e):
        return super().core(b, pos, step, e, s)


class CodaWithoutEntryNorm(OracleLM):
    """The coda entered without its ln_f (huginn_blocks.py:269)."""

    def coda(self, b, pos, s):
        x = s
        for i in range(self.c.n_coda):
            x = self.block(f"coda.{i}.", x, self.coda_base + i, b, pos)
        return K.linear_row(K.rmsnorm(x, self.w["ln_f"], self.c.norm_eps), self.w["lm_head"])


class StepLayerSlotsSwapped(OracleLM):
    """Core slot = n_prelude + layer * T_total + step (a transposed slot map)."""

    def slot_core(self, step, layer):
        return self.c.n_prelude + layer * self.c.T_total + step


MUTANTS = {
    "residual_after_norm": _mutant_block("residual_after_norm"),
    "swap_norm23": _mutant_block("swap_norm23"),
    "swap_gate_up": _mutant_block("swap_gate_up"),
    "mlp_residual_from_block_input": _mutant_block("mlp_residual_from_block_input"),
    "swapped_adapter_halves": SwappedAdapterHalves,
    "coda_without_entry_norm": CodaWithoutEntryNorm,
    "step_layer_slots_swapped": StepLayerSlotsSwapped,
}


def test_unmutated_block_restatement_agrees():
    """The restated block the mutants are built from passes every pin when
    unmutated, so each mutant differs from the oracle only by its slip."""
    plain = _mutant_block("none")
    assert all(pin(plain) for pin in PINS)


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_pins_catch_wiring_slip(name):
    cls = MUTANTS[name]
    assert not all(pin(cls) for pin in PINS), f"no pin catches the {name} slip"
