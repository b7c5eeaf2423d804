"""MI355X-native wavefront decode step (WFD) for looped language models.

Importable as `wavefront_decoding_amd` (the directory name carries a hyphen;
`__graft_entry__.load_package()` registers it under that name).

Layers, bottom-up:
  csrc/*.hip        hand-written gfx950 kernels behind the C ABI of include/wfd.h
  _lib, ops         ctypes binding + torch-tensor front end (no host fallback)
  attention         the reference's attention-backend API (attn_dense,
                    attn_cutoff_multi, attn_varlen, attn_varlen_q1_padded,
                    set_backend/backend, compute_qkv) on the HIP kernels
  kv_cache          StaticKVCache / BatchStaticKVCache over one flat device buffer
  model             synthetic looped-LM configs and seeded random-init weights
  engine            the device engine: P / R / C unions as fused launch
                    sequences, captured as hipGraphs (one replay per tick)
  blocks            P / R / C block forwards (single sequence and batch union)
  state, policy, acceptance, emu, batch_state
  scheduler         generate_wavefront_dynamic, generate_draft_then_verify
  scheduler_batch   generate_wavefront_batch, ar_generate_batch, generate_dtv_batch
"""
from __future__ import annotations

__all__ = ["__version__"]
__version__ = "0.1.0"
