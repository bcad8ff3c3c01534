"""CPU oracle for the fp4x decode GEMV path — TEST INFRASTRUCTURE ONLY.

A restatement, in numpy (and C for the order-exact sums), of the reference
plugin's quantize / dequantize / GEMV / mixer / fast-head semantics
(x/fp4x_kernels.py, x/fp4patch.py).  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg use it, to check results; the product path never
imports it.

Modules
  formats  number codecs: bf16, fp16, e4m3fn, e8m0, e2m1
  quant    the reference quantizers and dequantizers, plus an OCP-MX MXFP8
           quantizer (the reference receives MXFP8 pre-packed)
  gemv     dequantize-then-matmul GEMV semantics (fp32 accumulation)
  hc       hyper-connection mixer rounding points
  head     fast LM head and draft head flows (INT2 coarse -> top-C ->
           exact rescore); coarse sums are exact sums rounded to fp32
  ordered  C replica of the rescore kernels' fma order (bit-exact refined
           logits), float64 exact sums and the MFMA error bound

How each function is pinned (checked by tests/test_oracle_*.py):
  formats   exhaustive tables against closed forms and torch's float8/fp16
            dtypes; bf16 rounding against torch's bfloat16 cast
  quant     golden vectors written by running the reference's own torch
            quantizers in the build container (tests/golden/), tie cases,
            and invariants (round-trip error bounds, code ranges)
  gemv      brute force float64 sums on tiny shapes; dequant-equals-closed-form
  hc        closed forms (sigmoid exactly 1 at x >= 18, 0 at x <= -104, 1/2
            at 0) and exact rational arithmetic with a 200-bit sigmoid over
            dense bf16 sweeps; each dropped bf16 rounding is shown to fail
            (test_oracle_pins.py)
  head      top-C order against a brute-force lexicographic sort (bf16 and
            fp32 rows, ties, +-0, NaN, +-inf), with mutant key rules shown to
            fail; coarse sums against brute-force exact rational sums
  ordered   the fma order against a fold of exact rational fma steps on tiny
            inputs (a different lane split is shown to give other bits)

Parity unpinned: the reference's sigmoid is Triton's tl.sigmoid, whose fp32
rounding this container cannot run; the oracle (and the HIP kernels) use the
correctly rounded fp32 sigmoid.  The reference's tl.sum over the hc streams
leaves the order open; the oracle adds the streams in order, which equals any
order whenever the partial sums are exact in fp32.
"""
