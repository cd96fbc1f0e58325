"""CPU oracle for the NKIPy MI355X backend -- TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy, the reference's CPU path for the hot-path
kernels: the reference runs a kernel by calling the NumPy function directly
(README.md:118-133), so its CPU results are NumPy arithmetic on the kernel's
formula.  Each function cites the reference file:line it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the reference that results are compared
with or as the reported CPU baseline.
The product (nkipy_amd) never imports it.

Pins (tests/test_oracle.py):
  * softmax          -- the 2x2 golden vectors held in the reference's tutorial
                        notebooks; float64 brute force; rows sum to 1; shift
                        invariance.
  * rmsnorm          -- float64 closed form; scale invariance; linearity in w;
                        constant-magnitude rows give +-w.
  * swiglu / GEMM    -- float64 brute-force triple loop on tiny shapes; K = 1;
                        identity weights.
  * linear attention -- O(T^2) masked quadratic form in float64 (the chunked
                        recurrence must equal it exactly in exact arithmetic);
                        chunk = T reduces to the quadratic form.
  * bf16 / fp8       -- closed-form RNE rounding / E4M3FN decode cross-checked
                        against torch's conversions.
  * decoder layer    -- composed of the pinned parts above plus RoPE (pinned by
                        rotation-norm invariance and position 0 = identity) and
                        causal attention (pinned by a float64 per-query loop).
"""
