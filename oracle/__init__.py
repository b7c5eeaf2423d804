"""CPU oracle for the wavefront decode step -- TEST INFRASTRUCTURE ONLY.

A plain numpy / Python restatement of the reference's algorithm for the hot
path (per-depth slot KV caches, wavefront attention, the looped-LM block
forward, the WFD / sequential / batch schedulers), written to be obviously
correct rather than fast. Every function cites the reference file:line it
follows (paths relative to the reference checkout).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker / the timed CPU baseline. The
product path (wavefront-decoding_amd/) never imports it and has no CPU
fallback.

Pinning (how each part is checked against something other than itself;
tests/test_oracle_*.py):
  kernels.attention   torch SDPA with an explicit mask (library routine) on
                      small shapes; kv_len = 1 -> o = v0; identical keys ->
                      mean of V; GQA == MHA with repeated K/V.
  kernels.rmsnorm     torch.nn.functional.rms_norm.
  kernels.rope        complex multiplication by exp(i * pos * theta_j);
                      norm preservation; <rope(q,m), rope(k,n)> depends only
                      on m - n.
  kernels.swiglu      torch.nn.functional.silu composition.
  slots               closed-form slot formula, bijectivity over the layout.
  scheduler           golden counter/token traces written by the reference's
                      own batch scheduler (tests/golden/); WFD == sequential
                      tokens; T_draft == T_total == sequential call for call;
                      alpha = 1 -> no rejects; alpha = 0 -> every draft rejected.
  model (P/R/C)       the composition (tests/test_oracle_composition.py):
                      closed forms (Wqkv = fc = 0 -> norm_4(norm_2(x)); a
                      lone key returns its value, so a block at position 0 is
                      a fixed chain of library calls), the adapter's halves
                      ([I | 0] reads s, [0 | I] reads e), and a dense causal
                      formulation in torch over whole prompts (library
                      RMSNorm / linear / SiLU / SDPA, complex-number RoPE)
                      that must reproduce the per-slot oracle's logits and
                      slot caches; planted wiring slips (residual after the
                      norm, swapped norms, swapped adapter halves or gate/up,
                      a missing coda ln_f, a transposed slot map) each fail.
"""
