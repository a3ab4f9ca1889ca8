"""CPU oracle for the MoE-HLM expert layer -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of Yggdrasil's
MoE-HLM expert layer (``holograph/models/hlm_block.py:154-183`` and what it
calls).  It exists to check the HIP implementation in ``yggdrasil_amd``:

* only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
  ``bench.py`` may import it, and only as the checker / the timed CPU baseline;
* the product path (``yggdrasil_amd``) never imports it and has no CPU
  fallback -- it raises when the HIP library is missing.

Modules
-------
cl3      Cl(3,0) Cayley tables derived from the closed form, element-wise
         geometric product in the reference's term order, the 8x8
         left-multiplication expansion ``L(w)``.
moe      fp32-faithful NumPy restatement of CliffordLinear, the grade-wise
         activations, CliffordRouter, the dispatch counting sort, the combine
         and the whole ``_moe_forward``; plus the build-defined routing rule
         (descending top-k, lowest-index ties) and the int8 quantizer.
native   ctypes binding of the C restatement (``oracle/csrc/cl3_oracle.c``) and
         of ``oracle/_ref/libmjolnir_cpu.so``, the reference's own CPU
         geometric matmul compiled from ``/root/reference`` sources.

Parity pinning (what checks each function) is listed in the module docstrings;
a function with no independent check says "parity unpinned" there.
"""
