"""Oracle for the DDPM hot path.

THIS PACKAGE IS TEST INFRASTRUCTURE. It is what the product is tested against, never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package
(``dynamicconvolutionoperator_amd``) never imports anything from here, and its
GPU path raises when the HIP library is missing instead of falling back.

Contents
--------
``unfold_ref``  torch restatement of the reference's Unfold oracle
                (unfold_impl.py:5-42) plus closed-form backward formulas
                (triton_impl.py:94-132, _triton_kernels.py:430-811).
``c_oracle``    ctypes wrapper around ``ddpm_oracle.c``: an independent,
                loop-level double-precision restatement of the same maths,
                built by ``oracle/Makefile`` into ``oracle/libddpm_oracle.so``.

How each function is pinned (none is pinned by retyping its own formula):
* ``dynamic_cat`` / ``generator_dynamic_cat``: hand-checkable integer
  known-answer vectors in ``tests/golden`` written by a self-contained
  brute-force loop script; closed forms (K=1 gives ``k_d * x`` for every d,
  zero kernels give zero branches, a one-hot kernel gives a zero-padded
  shifted copy of x, ``cat[:, :C] == x``); agreement with the C restatement.
* ``dynamic_cat_backward`` / ``generator_dynamic_cat_backward``: torch
  autograd through the Unfold graph (a different code path: unfold's adjoint
  is fold), the integer known-answer backward vectors, the adjoint identity
  <J v, g> == <v, J^T g>, and the C restatement.
"""
