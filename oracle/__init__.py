"""CPU oracle for the block-sparse attention path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it,
and only to check results (or, for bench.py, as the timed CPU baseline).  The product
(polyhedral_amd) never imports it and has no CPU path.

  oracle.masks      predicates of gpu/masks_gpu.py:37-61 (+ PREFIX_LM, difference)
  oracle.blockindex gpu/blockindex.py:32-51 restated in numpy (small N) and the
                    streaming C builder (pa_oracle.c, any N)
  oracle.permute    gpu/permute.py:12-31 restated (argsort), row gather / scatter
  oracle.attention  gpu/reference.py:5-17 restated (float64, row chunked), the
                    kernel's online-softmax recurrence (tests/test_kernel_math.py:27-48)
                    and the log-sum-exp merge of a disjoint split

Pinning: every function is checked in tests/test_oracle_*.py against the
reference's recorded counts (tests/golden/reference_counts.json), closed forms,
brute force or textbook identities; none is checked only against a retyping of
itself.
"""
