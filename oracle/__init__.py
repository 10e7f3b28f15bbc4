"""CPU oracle for the TTL tile-op hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what tt-lang's functional simulator
(`python/sim`, the reference's only executable semantics) computes for the
tile programs the MI355X library runs.  Only `tests/`, `__graft_entry__.smoke()`
and `bench.py`'s `cpu_baseline` leg may import it, and only as the checker or
the timed CPU baseline; the product (`tt-lang_amd/`) never imports, links or
runs anything here.

Modules and what pins each function (the checks live in tests/test_oracle.py):
  tile_ops   op-level restatement: elementwise tile ops with per-op dtype
             rounding (python/sim/block.py:870-1010, ttnnsim.py:67-109,384-452),
             store(acc) (block.py:805-868), per-tile matmul + bf16 accumulation
             (block.py:1012-1013), SDPA in fp32 (spec ops only).
             Pinned by: the simulator's acc known answer (test/sim/test_cb.py:
             801-833), closed forms (bf16 RNE of an exact fp32 sum/product,
             broadcast identities), brute force against float64 on small
             inputs, softmax invariants.
  sim_exec   eager, tile-by-tile cooperative executor of unmodified @ttl.kernel
             programs (CB ring, zero-fill on reserve, row-major tile copies;
             python/sim/cb.py:302-408, copyhandlers.py:295-380,
             tensoraccessor.py:125-159, kernel.py:89-291).  Pinned by the
             reference examples' own torch goldens (eltwise_add.py:131-132,
             singlecore_matmul.py:84-88, multicore_matmul.py:159-160,
             broadcast.py:126-143) and the closed-form tile order of
             test/sim/test_copy.py:340-500.
  bfp8       bfloat8_b codec, C (bfp8_ref.c) plus an independent numpy
             restatement.  The reference fixes only the tile size (1088 B,
             python/ttl/dtype_utils.py:174-175); the format is defined by this
             build.  Pinned by brute force over every (exponent, sign,
             magnitude) byte triple against exact float64 arithmetic, hand
             computed vectors, and the C-vs-numpy cross-check.
"""
