"""CPU oracle for the ragged paged-attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``auto_infer_amd`` imports this package;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and there only as the checker (or the timed CPU
baseline), never as the product path.

Contents (each function cites the reference file:line it restates):

* ``oracle.pack``       -- BatchPlan -> device metadata (numpy/python loops):
  ``slot_mapping``, ``build`` (eager runner), ``decode_stage``,
  ``spec_decode_stage``, ``continuation_stage``, ``prefill_stage`` and the
  dirty-row block-table upload counter.
* ``oracle.paged_attn`` -- float32 torch-CPU restatement of the KV slot write
  and of the paged attention op (TND layout, bottom-right causal, GQA head
  mapping, absorbed-MLA latent variant), plus a float64 brute-force variant
  used to pin it.

Pinning status (what checks each function; see tests/test_oracle_*.py):

* pack.*            -- the reference's literal golden vectors
  (tests/golden/*.json, transcribed from the reference's own tests).
* paged_attn.*      -- float64 brute force on tiny inputs, the closed forms
  Lq == Lk (dense causal, pinned like the reference's
  ``dense_causal_attention`` test) and Lq == 1 (plain softmax), block
  permutation invariance and request isolation.  The vendor op the reference
  calls (torch_npu FIA) is closed and absent, so no reference vector exists
  for attention values: the north-star float32 gather-softmax *is* the
  oracle.
* kv_write          -- closed form (index assignment), untouched-slot
  invariance.
"""
