"""CPU oracle for the paged-KV speculative verify path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference engine's semantics for the
path the HIP library implements:

* ``oracle.kv_pool``   -- block allocator + paged KV cache (engine/kv.py:41-224)
* ``oracle.attention`` -- gather_ctx / GQA expansion / paged extend attention
                          (engine/attention.py:32-93, 170-216)
* ``oracle.sampler``   -- logits_to_probs, acceptance_probability,
                          residual_distribution, sample_token, batch_accept
                          (specdec/sampler.py:16-99, engine/spec_scheduler.py:41-88)
* ``oracle.spec_step`` -- the per-sequence commit / rewind rule of a spec round
                          (engine/spec_scheduler.py:269-322)

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only to check results (or as the timed
CPU baseline). The product path (``speculative-decoding-lab_amd``) never imports it
and has no CPU fallback.

Pinning status (what checks each function against something other than its own
formula) is listed in each module's docstring; every function here is pinned by
a test under ``tests/test_oracle_*.py``.
"""
