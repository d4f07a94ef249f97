"""CPU oracle of the softhier-ops hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (and in plain C, sh_oracle.c), what the reference computes on the path
`sh_gemm / sh_attention / sh_layernorm / sh_softmax_rows / sh_gelu / sh_add / sh_add_bias / sh_scale /
sh_transpose` and its test protocol, following these reference files (runwangdl/softhier-mlir):

  - softhier_mlir/testing/lcg.py:13-106 and runtime/sh_test.inc.c:2-51  -> oracle.lcg
  - runtime/sh_rt.inc.c:31-59 (fp16 codec)                              -> oracle.fp16, sh_oracle.c
  - tests/gvsoc/run.py:116-121, 152-158, 921-934                        -> oracle.refs (gemm, row ops, attention)
  - softhier_mlir/testing/siglip_ref.py:9-45, frontend/siglip.py:133-168 -> oracle.refs (encoder layer)

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import it, and only as
the checker (or the timed CPU baseline): the product path (softhier_mlir_amd) never imports, calls or links
anything here, and fails loudly when its HIP library is missing.

How each function is pinned (tests/test_oracle_*.py): the LCG by the sample positions of the reference's
committed device log (tests/golden) and its leapfrog == scalar self-test; fill values and the attention
restatement by the 512 logged attention outputs; the fp16 codec exhaustively against numpy's IEEE
conversion and the C restatement; GEMM by exact small-integer products, a triple-loop brute force and the
reference's known answers (X = 1, W = 1/1024 => Z = 1; Z0 = 3 accumulate); row ops by closed forms
(two-element layernorm, constant rows, softmax invariances, the erf-GELU bound) and brute force; the
encoder layer by zero-weight closed forms and its composition of the pinned ops. Parity of numpy's own
BLAS summation order is unpinned (no reference vector holds full-precision GEMM outputs).
"""
