"""`ttl.utils`: the reference installs its python/utils package here
(imported as ttl.utils.block_allocation by its hardware tests and metal
examples)."""
