"""CPU oracle for the llmlab decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU and in plain PyTorch, what the reference
computes on the hot path (each function cites the reference file:line it
follows). It is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. Nothing in ``systems_for_llms_amd`` imports it, and the product path
raises when its HIP library is missing instead of falling back here.

Pinning (what fixes each function independently of its own formula):

* ``model.forward``: golden logits written by the reference ``TransformerLM``
  itself (``tests/golden/make_golden.py``), the config-1 greedy token sequence
  from the same source, the reference's causal-prefix invariance.
* ``model.rope_tables``: bit-exact against the reference's buffers (golden hash).
* ``model.greedy_cached`` / ``KVCacheOracle``: the golden 192-token sequence;
  KV-cached == recompute.
* Storage-format floors (``round_weights``, ``kv_dtype``, ``act_dtype``): not
  reference behaviour but bounds on what bf16 storage alone changes; pinned by
  chunked-cache == full-forward under the same formats, by fp32 formats being
  exact no-ops, and by each rounding point moving the logits (a dropped
  rounding fails a test).
* ``attention.decode_reference``: equality with ``F.scaled_dot_product_attention``
  on explicitly repeated KV heads with a length mask, as the reference's tests do.
* ``attention.masked_attention``: fp64 agreement with SDPA under the dense mask;
  the dense mask against the reference's known-answer schedule and brute force.
"""
