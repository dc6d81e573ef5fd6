"""Oracle for the attention block — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or the timed CPU baseline),
never as part of the product path.

Contents
  block.py        fp32/fp64 CPU restatement of the reference's eager block
                  (README.md:42-64) with torch library routines; autograd
                  gives its gradients.
  exact_bwd.py    independent numpy restatement of the block's exact
                  backward (hand-derived, brute-force attention), plus the
                  reference's rotated-space q/k shortcut
                  (fast_triton_attn.py:603-634) for comparison.

Pinning (tests/test_oracle.py): each function is checked against library
routines, closed forms, invariants, brute force and finite differences;
the reference ships no golden vectors or tests of its own (it has two files
and no test directory), and its Triton/ATen path needs a GPU, so it cannot
be executed here. The committed fixture tests/golden/block_t16.npz
regression-locks the oracle's outputs on a tiny case.
"""
