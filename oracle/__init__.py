"""CPU oracle for the paged attention path (TEST INFRASTRUCTURE ONLY).

This package restates, on the CPU with PyTorch/numpy, the algorithms of the
reference (lv76/mini-llm-runtime) that the HIP library replaces. Each function
cites the reference file:line it follows. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the reference to compare against or as the timed CPU
baseline; the product package ``mini_llm_runtime_amd`` never imports it and
never falls back to it.

Modules
- ``paged_attention``: decode (single request, per-request loop, tensorized
  batch), chunk prefill (dense reference and tiled online softmax).
- ``paged_kv_cache``: block pool, LIFO allocator, slot-mapping write.
- ``slots``: slot/block-table construction of the ModelBatch builder.
- ``textbook``: float64 numpy attention with explicit masks, used to pin the
  restatements above (it follows no reference code: it is the definition).

Pinning (see tests/test_oracle_pins.py): the decode and chunk restatements are
checked against the reference's stored masked-SDPA known answer
(tests/golden/sdpa_known_answer.npz, copied from the reference's
tests/model/snapshots), against the float64 textbook attention on paged
layouts, and against each other the way the reference's own tests check them;
planted mistakes (wrong GQA map, dropped scale, off-by-one causal mask,
ignored padding) must fail those checks. The KV write is pinned by its closed
form and the allocator by the reference tests' assertions.
"""
