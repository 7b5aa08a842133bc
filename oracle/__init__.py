"""CPU oracle for the weighted_abs_sum / weighted_laplace_sum hot path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only as the checker
(or, for bench, as the timed CPU baseline) -- never as a product code path. The product (libqlka.so behind the
weighted_abs_sum / weighted_laplace_sum packages) has no CPU fallback.

Modules:
  brute.py   fp64 brute-force restatement of every boundary function (direct O(M*N*D*C) sums), the sort / merge-rank
             contracts, and an independent sorted-prefix formulation used to pin the brute force.
  dense.py   torch-CPU restatement of the reference's own PyTorch path (Experiments/kernel_attention/kernels.py:68-89,
             attention.py:32-50,67-92) used as the CPU baseline and as the "reference PyTorch path" parity target.
  inputs.py  seeded generators for the five BASELINE.json configurations.

Parity status of each function (what pins it) is listed in brute.py's docstring.
"""
