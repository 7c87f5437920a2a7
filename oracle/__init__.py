"""CPU oracle for the GPTQ / GPTAQ / G2PTQ per-layer quantization path.

TEST INFRASTRUCTURE ONLY.  This package is a torch-CPU fp32 restatement of the
reference arithmetic, written in the reference's own operation order so that it
can serve as the checker for the HIP implementation in ``g2ptq_amd``.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package never imports, links or runs
anything from here.

Every public function cites the reference file:line it restates.  Paths are
relative to the reference repository root (G2PTQ/G2PTQ).

Pinning (what checks each function independently of its own formula) lives in
``tests/test_oracle_*.py``:

* quantizer (``quant``): closed-form known answers, half-to-even ties, the
  all-zero group, and the reference test's "unified asym == fake_quantize"
  equivalence;
* Hessians (``hessian``): fp64 brute force ``(2/n)·XᵀX``, symmetry/PSD,
  streaming == one-shot, saliency≡1 relations;
* factor (``factor``): ``UᵀU == (H + λI)⁻¹`` against fp64 LAPACK, uniqueness of
  the positive-diagonal upper factor, forced damp-retry path;
* compensation (``compensate``): the GPTQ identity ``W − Q = E·U``, diagonal U
  ⇒ RTN, blocksize invariance, GPTAQ(P=0) == GPTQ, G2PTQ(β=0) == GPTQ, a tiny-C
  fp64 optimal-brain-surgeon brute force, and the reference test's
  pre-refactor loops restated independently in ``original_loops``;
* trust region (``flows.g2ptq_trust_region``): β∈[0,1], β=0 at α=0,
  ``GHinv == β·Grad·A⁻¹``, a 1×2 case worked by hand, and a diagonal A whose
  β, Z and GHinv reduce to a scalar closed form (with and without the clamp).
"""
