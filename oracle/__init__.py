"""CPU oracle of fastmoe's grouped weighted scatter-add -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker (or the timed CPU baseline); the product path
(``fastmoe_amd``) never touches it.

Contents
  * ``cref``      -- ctypes wrapper of ``combine_ref.c``: the scalar C restatement of the
                     reference's CPU algorithm (src/fastmoe/kernels/ops.py:373-384 forward,
                     :344-353 backward, :233-268 metadata) plus the token-major plan.
  * ``torch_ref`` -- the same algorithm written with torch CPU ops exactly as the reference runs
                     it (cat/mul/index_add_, index_select/mul/split), plus an fp64 autograd gate
                     gradient.  It pins ``cref`` and is the timed CPU baseline.

Parity pinning (tests/test_oracle.py): cref vs torch_ref bit for bit in fp32; both vs brute-force
Python loops on small inputs (the form of tests/test_cpu_moe.py:94-114 in the reference);
closed forms and invariants -- linearity in w (w -> 2w doubles out exactly), a k=1 permutation is
an exact scatter, all-ones inputs count multiplicities, empty experts add nothing, any split of
the packed rows into experts gives the same bits, grad_w equals the fp64 autograd gradient, the
plan equals a stable argsort of idx -- and the committed golden fixtures under tests/golden/.
"""
