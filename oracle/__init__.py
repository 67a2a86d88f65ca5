"""TEST INFRASTRUCTURE ONLY: CPU oracle for the op1/op4 hot path.

This package restates the reference algorithms on the CPU so that tests, the
smoke check and the benchmark's CPU-baseline leg can check the HIP library.
Nothing in ``treemoe_spec_amd`` imports it; the product path has no CPU
fallback.

* ``oracle.oracle_c``  — ctypes front end of ``c/tm_oracle.c``: bit-exact
  statement of routing, gates, demand, layouts, argmax, greedy walk and KV
  commit (fixed order of IEEE fp32 operations).
* ``oracle.op1_ref``   — torch restatement of ``treemoe/ref/tree_moe_ref.py``
  and of the padded layout of ``treemoe/kernels/op1_tree_moe.py:66-149``; the
  FP32/FP64 expert-FFN golden.
* ``oracle.op4_ref``   — restatement of ``treemoe/ref/verify_ref.py`` and of
  ``PagedKVCache.commit_tree`` (``treemoe/model/kv_cache.py:88-106``) for any
  page size.

Parity unpinned: the exact bf16 bits of the router logits.  The reference takes
them from torch's ``F.linear`` (treemoe/ref/tree_moe_ref.py:83), whose
reduction order torch does not fix.  The oracle fixes one order (64 lane
partials, xor fold); the tests pin each logit to within one bf16 ulp of the
FP64 dot product and the gates to torch's ``softmax(F.linear)`` within 2e-6,
which bounds but does not fix the bits.  Every other function is pinned by the
reference's known-answer tests, brute force or closed forms (tests/test_oracle_*.py).
"""
