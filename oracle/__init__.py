"""CPU oracle for the quantized-weight matmul path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference's CPU definitions of the GGUF dequantizers,
weight layouts and GEMV/GEMM semantics (each function cites the reference file:line it
follows).  It is the checker: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product path
(``thunderllamax_amd``) never imports, calls or falls back to anything here.

Pinning status (how each function is checked, see ``tests/test_oracle_*.py``):

* ``quants.dequant_iq3xxs_*``  -- three independent restatements of the reference agree
  bit-for-bit (numpy packed-row form, numpy raw-block form, CUDA per-lane form), plus
  closed-form known-answer blocks.  The *content* of the IQ3_XXS grid table is pinned only by
  invariants + SHA-256 (third-party table, absent from the reference).
* ``quants.dequant_q6k*``      -- numpy form vs two CUDA per-lane forms (h6k2048, aq6k8),
  plus known-answer blocks.
* ``quants.dequant_iq4xs*``    -- numpy form vs CUDA per-lane form (gx8e256up4), plus
  known-answer blocks; ``KVALUES_IQ4NL`` content pinned by invariants + SHA-256.
* ``layouts``                  -- packers vs their own byte-exact inverses.
* ``gemv``                     -- float64 matmul of the dequantized values (the math fixes
  this); ``hsilu16`` over all 63,488 finite fp16 inputs against float64 silu within the
  first-order bound of its five fp16 roundings, its exp2 overflow (-0) and underflow
  (identity) branches exactly, and planted mistakes that the bound must catch;
  ``swiglu16`` by its algebra (u = 0, 1, -u, 2u) and against float64 silu(g) * u
  (tests/test_oracle_gemv.py).
"""
