"""MI355X-native wavefront decode step (WFD) for looped language models.

Importable as `wavefront_decoding_amd` (the directory name carries a hyphen;
`__graft_entry__.load_package()` registers it under that name).

Layers, bottom-up:
  csrc/*.hip        hand-written gfx950 kernels behind the C ABI of include/wfd.h
  _lib, ops         ctypes binding + torch-tensor front end (no host fallback)
  attention         the reference's attention-backend API (attn_dense,
                    attn_cutoff_multi, attn_varlen, attn_varlen_q1_padded,
                    set_backend/backend) routed to the decode kernel
  kv_cache          StaticKVCache / BatchStaticKVCache over one flat device buffer
  model             synthetic looped-LM configs and seeded random-init weights
  blocks            P / R / C block forwards (single sequence and batch union)
  state, policy, acceptance, emu, batch_state
  scheduler         generate_wavefront_dynamic, ar_generate
  scheduler_batch   generate_wavefront_batch, ar_generate_batch
  graph             hipGraph step engine (captured decode ticks)
"""
from __future__ import annotations

__all__ = ["__version__"]
__version__ = "0.1.0"
