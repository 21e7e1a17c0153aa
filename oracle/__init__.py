"""CPU oracle for the DSCQuant W4A4 linear-layer path.

TEST INFRASTRUCTURE ONLY.  This package is the reference the HIP product path
(``dscquant_amd``) is compared against.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it; the product never does, and never falls back to it.

Contents
--------
``dscq_oracle.c`` / ``native.py``
    Plain-C restatement (IEEE fp32, round-half-even, no fma contraction) of
    the reference's quantization rules (core/quantization.py:4-45), the W4A4
    extension's padding/packing/GEMM/epilogue (kernel/w4a4.cu:20-161) and the
    block-Hadamard rotation fold (core/linear.py:34-37 rule).
``numpy_ref.py``
    An independent vectorised numpy restatement of the same rules, used to
    cross-check the C code and for cases where a vectorised form is handier.
``fakequant.py``
    A torch-CPU restatement of ``QuantLinear.forward`` with ``enabled=True``
    (core/linear.py:48-52): the reference's CPU fake-quant path, timed as the
    CPU baseline.

Every function cites the reference file:line it follows.  All functions are
pinned by tests/test_oracle.py (closed forms, ties, invariants, exhaustive
nibble tables, brute-force integer GEMM, dense Hadamard).
"""
