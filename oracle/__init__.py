"""CPU oracle for the paged-attention path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference's own algorithm for the hot
path so the HIP kernels can be checked against it:

  paged_attention_ref   reference nanoserve/attention.py:99-190 (gather + SDPA)
  dense_reference       reference tests/test_paged_attention.py:24-36 (fp64 textbook)
  reshape_and_cache_ref reference nanoserve/kv_cache.py:73-81 (.to() + index_copy_)
  slot_mapping_ref      reference nanoserve/block_manager.py:131-132 (closed form)
  rope.*                reference nanoserve/layers.py:65-90 (rotary table and
                        apply) and qwen2.py:53-57 (rotary, then cache write);
                        pinned in tests/test_oracle_rope.py

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it, and only as the checker (or the timed CPU baseline), never as the
thing measured or shipped.  The product package nanoserve_amd never imports it.

Parity pinning (each function is checked by tests/test_oracle.py):
  paged_attention_ref   against dense_reference on the reference's own test
                        cases, closed forms (one key, identical keys, zero
                        query), a hand-written scalar softmax on tiny inputs,
                        and invariants (table permutation, stale-slot
                        poisoning, chunked == whole prefill).
  dense_reference       against closed forms and the scalar softmax.
  reshape_and_cache_ref against numpy's independent float16 rounding and an
                        integer bfloat16 rounding on random and special
                        values, known-answer bit patterns, and slot formula.
  slot_mapping_ref      against brute-force per-token enumeration and the
                        reference test expectations.
The reference ships no golden vectors for this path; tests/golden holds small
fixtures written by this oracle (tests/golden/make_golden.py) as a regression pin.
"""
