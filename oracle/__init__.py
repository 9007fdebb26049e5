"""CPU oracle for ferrite's three kernels — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference's kernels and
of their jnp references (anxnd2211/ferrite-tpu, src/ferrite/kernels/*.py). It
is the checker the HIP kernels are compared against. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and only
as the checker or as the timed CPU baseline; the product path
(ferrite-tpu_amd/ferrite) never imports it and has no CPU fallback.

Modules:
  bf16       round-to-nearest-even f32 -> bf16 (the dtype casts of the reference)
  rmsnorm    rmsnorm.py:39-56 (kernel) and :193-199 (rmsnorm_reference)
  attention  flash_attention.py:370-380 (materialised oracle) + logsumexp,
             FA-2 analytic backward (:184-243, :326-330), and a blockwise
             restatement of the Pallas kernels' online softmax (:91-127)
  matmul     matmul.py:27-86 (blocked, zero-padded) and :129-131 (reference)

How each function is pinned (tests/test_oracle.py):
  bf16.round_bf16          torch's bf16 cast on CPU (library RNE), special values
  rmsnorm.*                closed forms (constant rows), the identity mean(xhat^2) = 1
                           at eps = 0, scale invariance, bit-exact h = bf16(x + r)
  attention.forward        pure-Python brute force (math.exp loops) on tiny inputs,
                           closed forms (row 0 = v[0], constant V, q = 0 -> uniform
                           weights and lse = log(i + 1)), prefix and key-permutation
                           invariance
  attention.backward       torch.autograd of a float64 torch attention (independent
                           derivation) and central finite differences
  attention.flash_*        the materialised forward/backward above
  matmul.*                 numpy's float64 product, identity matrices, exact
                           integer-valued products for the padded/blocked restatement
Parity unpinned: the bit-level rounding of XLA:CPU's exp/rsqrt and dot reduction
order inside the reference's jnp functions (jax is not installed anywhere this
build runs); the stated tolerances absorb them.
"""
