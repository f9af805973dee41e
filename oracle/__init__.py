"""
oracle — CPU fp64 restatement of the reference's hot-path algorithm, used ONLY as a checker.

This package is test infrastructure.  Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only to check or time against; the product (``mace_hip_kernels``) never imports it
and has no CPU fallback.

Modules and what each restates (reference file:line):
  * ``wigner``  real Wigner-3j symbols from sympy's exact Clebsch-Gordan coefficients carried into e3nn's real basis,
                real spherical harmonics from scipy's complex ones, Wigner-D matrices of that basis.  These pin the
                coefficient tables the reference probes from e3nn (conv.py:74-86).
  * ``conv``    the interaction convolution: unfused ``scatter_sum(TP(x[sender], Y, W), receiver)`` from dense CG
                tensors, and the fused per-term formulas of the three kernels (conv.py:109-141 forward,
                144-176 d/dx, 179-222 d/dW and d/dY), plus the CSR builder (conv.py:229-235).
  * ``sc``      the symmetric contraction: dense Σ_ν U_ν·W_ν·x^⊗ν evaluation (the math of symmetric.py:1-13), the
                symmetrised polynomial table (symmetric.py:20-75) and its evaluation/derivative (symmetric.py:82-131).
  * ``neighbours`` the graph the convolution's CSRs are built from (conv.py:229-235): the periodic neighbour list in
                MACE's edge convention and the fixed-size padded layout the reference recommends (README.md:77-78).

Which check pins which function is listed in each module's docstring.
"""
