"""CPU oracle for the paged mixed-precision KV-cache hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product imports this package: only
`tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`
may, and only as the checker (or, for `cpu_baseline`, as the CPU path timed
beside the GPU). The product path is the HIP library; it fails loudly when that
library is missing and never falls back to anything here.

Each function restates, in NumPy, the arithmetic of the reference
(lecuong1502/Semantic-Aware_Adaptive_KV_Cache_Precision, "MicroInfer") and
cites the reference file:line it follows. How each function is pinned
(known answers from the reference's own tests, closed forms, invariants,
brute force on tiny inputs) is listed per module; see `PINNED` in each.

Modules:
  quant      page layout, scale_of, code_of, quantise/dequantise a page
  attention  float64 attention (contiguous, causal paged over tiers), per-page mass
  ewma       the importance-score EWMA in fp32, in the device's order
  slots      the tail-swap page allocator and its granule accounting
  pointwise  RoPE, RMSNorm, SwiGLU float64 references
  dense      float64 projection with its term magnitudes, embed, argmax
"""
