"""CPU oracle for the verify step -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the checker (or the timed CPU baseline); the product path (snowllm_amd) never
imports it. Modules:

  accept       ctypes binding of accept.c: argmax, spec_accept, softmax, top-k/top-p,
               rejection sampling, sampling pick -- canonical arithmetic, bit-exact target.
  quant        GGUF Q4_K / Q8_0 block generators, decoders and fp64 GEMV.
  reference    torch restatements of the reference's own CPU semantics (reference_reject,
               target probabilities, dense attention), used to pin the oracle.
"""
