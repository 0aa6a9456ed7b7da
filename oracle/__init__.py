"""CPU oracle for the quantized Conv/Gemm/MatMul integer path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package
(``quantanything_amd``) imports this package; only ``tests/``, the smoke check
in ``__graft_entry__.py`` and the CPU-baseline leg of ``bench.py`` do, and
only as the checker or the timed CPU baseline.

Contents:

* ``abi``      -- ctypes binding of a library exporting the 17 ``qa_*``
                  symbols of the reference C ABI, with wrappers restating the
                  reference ``quantization/native.py`` wrapper semantics.
                  Drives ``libqa_oracle.so`` (this repository's C restatement,
                  ``qa_oracle.c``) and ``_ref/libqa_ref.so`` (the reference's
                  own kernels compiled from source by ``Makefile``).
* ``twins``    -- NumPy restatement of the reference's NumPy twins
                  (``native.py:177-203``, ``:219-235``, ``:260-277``,
                  ``:377-556``), an independent second path.
* ``pipeline`` -- restatement of the integer-only inference path
                  (``quant_layers.py`` integer paths and ``prepare``,
                  ``quant_container.py:135-193``) over a graph and a q.json.

Parity pins (which check covers which function) are listed in each module's
docstring; every function is pinned by golden vectors from the compiled
reference (``tests/golden/``) or by closed forms / known-answer tests taken
from the reference's own test-suite.
"""
