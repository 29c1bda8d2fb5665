"""CPU oracle for the TaoMate-HD streaming attention hot path.

TEST INFRASTRUCTURE ONLY.  This package restates, on the CPU, the arithmetic
of the reference path so the HIP implementation can be checked against it.
Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
bench.py may import it, and only to check results or as the timed CPU baseline;
the product package (``taomate_hd_amd``) never imports it and has no CPU
fallback.

Modules
  bf16       bit-exact bf16 <-> fp32 conversion (round to nearest even)
  quant      INT8 quantizers (token, weight, smooth-K block), exact int GEMM,
             scaled-mm epilogue
  attention  fp64 softmax attention, torch-SDPA CPU restatement, INT8-QK
             attention emulation
  stream     the streaming hook, KV cache and session semantics on CPU

Every function cites the reference file:line it restates.  How each one is
pinned (closed forms, invariants, brute force, hand-derived cases) is listed
in tests/test_oracle.py; a function without such a check says
"parity unpinned" in its docstring.
"""
