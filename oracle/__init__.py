"""CPU oracle for the block-scaled FP8/FP4 GEMM family.

TEST INFRASTRUCTURE ONLY.  This package is the checker, never the product: only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import it.  The ``deep_gemm`` package never routes a call through here; if its
HIP library is missing it raises instead of falling back to the CPU.

It restates, in plain CPU torch / numpy, the reference's own reference math:

* ``quant``   -- UE8M0 rounding, e4m3 / e2m1 quantisation and decoding, and the
                 seeded operand generators (``tests/generators.py`` in the reference).
* ``layout``  -- the scale-factor layout contract of
                 ``transform_sf_into_required_layout`` (``tests/test_layout.py:39-50``)
                 and the psum / m_indices helpers (``tests/generators.py:212-235``).
* ``gemm``    -- dequantise-to-fp32 then matmul then cast (``tests/generators.py:320-322``),
                 grouped, masked, batched, K-grouped and einsum variants, and ``calc_diff``
                 (``tests/utils.py:36-43``).
* ``epilogue`` -- stochastic bf16 rounding (``tests/utils.py:70-92``) and FP8 output
                 quantisation (``tests/test_einsum.py:70-86``).

Every function is pinned by ``tests/test_oracle.py`` against closed forms, library
routines, brute force on tiny inputs and the committed fixtures in ``tests/golden/``.
Parity status per function is listed in each module's docstring.
"""
from . import quant, layout, gemm, epilogue  # noqa: F401
