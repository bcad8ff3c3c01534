"""CPU oracle for the fp4x decode GEMV path — TEST INFRASTRUCTURE ONLY.

A restatement, in numpy (and C for the order-exact sums), of the reference
plugin's quantize / dequantize / GEMV / mixer / fast-head semantics
(x/fp4x_kernels.py, x/fp4patch.py).  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg use it, as the checker; the product path never
imports it.

Modules
  formats  number codecs: bf16, fp16, e4m3fn, e8m0, e2m1
  quant    the reference quantizers and dequantizers, plus an OCP-MX MXFP8
           quantizer (the reference receives MXFP8 pre-packed)
  gemv     dequantize-then-matmul GEMV semantics (fp32 accumulation)
  hc       hyper-connection mixer rounding points
  head     fast LM head flow (INT2 coarse -> top-C -> exact MXFP8 rescore)
  ordered  C replica of the kernels' summation order (bit-exact sums)

How each function is pinned (checked by tests/test_oracle_*.py):
  formats   exhaustive tables against closed forms and torch's float8/fp16
            dtypes; bf16 rounding against torch's bfloat16 cast
  quant     golden vectors written by running the reference's own torch
            quantizers in the build container (tests/golden/), tie cases,
            and invariants (round-trip error bounds, code ranges)
  gemv      brute force float64 sums on tiny shapes; dequant-equals-closed-form
  hc        closed-form values at sigmoid special points; brute force
  head      top-C set identity against a full sort; exact-sum properties
  ordered   against float64 sums (error bound) and numpy sequential folds
"""
