"""CPU oracle for the quantized DiT-block hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this
directory. It is imported by ``tests/``, by ``__graft_entry__.smoke()`` (as the
checker of one small GPU invocation) and by the ``cpu_baseline`` leg of
``bench.py`` (timed as the reference's CPU path). It is never the thing
measured as GPU throughput and never a fallback for the HIP path.

Modules:

* ``cpu_ref``   -- torch-CPU restatement of the reference's eager backend
                   (``comfy_kitchen/backends/eager``), op for op, calling the
                   same torch CPU routines the reference calls
                   (``torch._int_mm``, ``F.gelu``, ``F.rms_norm``).
* ``npref``     -- independent numpy restatements of the integer/byte parts
                   (row quantizer, int GEMM, W4 decode, W4 weight generator),
                   written from the closed-form rules, used to pin ``cpu_ref``.
* ``c/``        -- the same integer rules in plain C (``liboracle.so``), a
                   third, language-independent restatement used by the tests.

Parity pinning status per function is listed in the header of each module.
"""
