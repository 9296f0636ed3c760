"""CPU oracle for the algebraic attention and fused algebraic head (TEST INFRASTRUCTURE).

This package is a NumPy restatement of the reference's dense (non-Pallas) algorithms
for the two hot kernels, used only as the checker:

* ``tests/`` compare the HIP path against it,
* ``__graft_entry__.smoke()`` checks one small HIP invocation against it,
* ``bench.py`` times it as the ``cpu_baseline`` leg.

Nothing in the product path (``algebraic-transformer_amd/``) may import it; the product
fails loudly when the HIP library is missing instead of falling back here.

Modules
-------
``numerics``   rho / int_pow / inv_root / bf16 rounding (algebraic.py:31-51, flash.py:76-114)
``attention``  dense and kernel-faithful attention forward/backward
               (algebraic.py:186-216, flash.py:189-361, 630-729, 823-857)
``head``       lean algebraic likelihood head forward/backward
               (algebraic.py:277-319, model.py:211-231, fused_head.py:72-275)
``closed_form`` independent float64 closed forms (softmax of compressed logits, torch
               autograd of the true NLL) that pin the functions above.

Parity status: every function above is pinned by a closed form or an independent
autodiff check in ``tests/test_oracle.py`` (see each function's docstring for the pin).
"""
