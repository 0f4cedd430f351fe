"""CPU oracle for the FlashAttention-2 forward path (TEST INFRASTRUCTURE ONLY).

This package restates, on the CPU, the semantics of the reference's forward
attention path (luyanaa/flash-attn-triton) so that the HIP kernels can be
checked against it.  It is the checker, never the thing measured or shipped:
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import it.  The product path (``flash_attn_triton``) never imports it and
fails loudly when the HIP library is missing.

Modules
-------
``attention``  float64 numpy restatement of the dense / cross / varlen /
               KV-cache semantics (``flash_attn_interface.py:15-49`` and the
               kernel epilogue rules of ``attention_kernel.py:275-533,27-104``).
``quant``      bit-exact float32 numpy restatement of the INT8 per-token
               quantizer (``attention_kernel_int8.py:27-39,58-79``) and the
               INT8-QK attention built on it (``attention_kernel_int8.py:82-217``).
``quant_int8.c`` an independent plain-C restatement of the same quantizer,
               compiled by ``oracle/Makefile`` and used to cross-check ``quant``.

Every public function here is pinned by tests in ``tests/test_oracle.py``:
against torch's CPU ``scaled_dot_product_attention`` (the oracle the
reference's own tests use, ``tests/test_compare_implementations.py:31-41``),
against closed forms (uniform attention, a single visible key, empty rows,
saturated softcap), against a pure-Python brute force on tiny shapes, and for
the quantizer against exact rational arithmetic and the C restatement.
"""
