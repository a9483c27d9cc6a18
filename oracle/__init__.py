"""CPU oracle for the real-quant MoE expert path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what lcj1111/RobustGEMQ computes on its
real-quant MoE path, so that the HIP kernels in ``robustgemq_amd`` can be
checked against it.  It is imported only by ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``, and
only as the checker: the product path never imports, links or calls it, and
fails loudly when its HIP library is missing instead of falling back here.

Modules (each function cites the reference file:line it restates):

* ``oracle.fp``      -- IEEE fp16 / bf16 per-op arithmetic as torch applies it
                        (compute in fp32, round to nearest even).
* ``oracle.quant``   -- RTN quantizer, fake-quant dequant, GemLite/HQQ packed
                        word layout, the build layout the kernels read.
* ``oracle.route``   -- router logits in the kernels' fixed fp32 order (C,
                        ``oracle/router_exact.c``), softmax / top-k /
                        renormalisation, the stable token->expert permutation.
* ``oracle.moe``     -- the per-expert dequantize-then-matmul loop in fp32
                        (the "fp32 reference") and the routed+shared combine.

How each function is pinned (golden vectors do not exist in the reference;
its tests draw inputs live on CUDA):

* RTN quantizer, dequant: exhaustive / sampled comparison with torch's own
  fp16 CPU arithmetic running the reference formulas, plus closed forms
  (grid round trips, constant groups, the 1-bit rule) -- tests/test_oracle.py.
* Packed layout: single-bit brute force over every code position for
  b = 1..4 (including the 3-bit tail and dead bits) and round trips.
* Router logits: exact for integer-valued inputs in any order, one-hot
  inputs select a weight column exactly, and the error bound of a length-H
  fp32 dot product against exact rational arithmetic.
* Top-k / softmax: brute-force enumeration on small E, scipy.special.softmax.
* Permutation: a literal loop over (expert, slot, token) as
  ``torch.where(expert_mask[e])`` orders it, compared with the sort.
* Expert loop: dense special cases that reduce to one matmul (all tokens on
  one expert, k = E) and the einsum formulation of the reference's
  Fused*MoEBlock.forward.

No function here is left "parity unpinned".
"""
