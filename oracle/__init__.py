"""CPU oracle of the BF16 projection path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only to check results (or as the timed CPU baseline).  The
product path (leanstack_amd) never imports it and has no CPU fallback.

Modules
  projections  CPU torch restatement of the reference's eager projection
               arithmetic (src/leanstack/runtime/qwen_explicit.py,
               src/leanstack/runtime/cutile_logits.py), bf16 in/out exactly as
               the reference computes it.
  brute        float64 numpy brute force of the same functions, written
               independently of torch, used to pin `projections`.
  packing      pure-numpy restatement of the packed tile layout (index
               arithmetic, no torch), used to pin the packers.

How each function is pinned (tests/test_oracle.py, tests/test_golden.py):
  - brute-force float64 agreement within bf16 rounding plus the fp32
    accumulation bound, on tiny and medium shapes;
  - one-hot activations reproduce a weight column exactly; power-of-two
    scaling is exact; rows are independent (M stacked GEMVs = one GEMM);
  - one-hot weight rows pin the [q|k|v] and [gate|up] segment order;
  - SiLU closed forms (silu(0) = 0, large +g -> g, large -g -> 0);
  - argmax: a planted unique maximum, and ties resolve to the lowest index;
  - committed golden vectors under tests/golden/ (float64 expectations).
Unpinned: the torch.compile/Inductor-fused numerics of the reference's
wrapped helpers (qwen_explicit.py:578-604, :963-971) and the cuTile kernels'
exact fp32 summation order (cutile_logits.py:27) -- neither runs without an
NVIDIA GPU and cuda.tile; the eager semantics are the oracle.
"""
