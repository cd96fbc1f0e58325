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
  * Qwen3 forms      -- the bf16 softmax steps, the bf16-step RoPE, the head
                        prologue, decode and prefill attention with their cast
                        points, and greedy sampling: each against torch's
                        op-by-op evaluation on bfloat16 tensors (bit for bit
                        where no fp32 sum is involved); decode attention
                        without casts equals the last row of causal attention.
                        The decode layer is composed of these parts.

Parity unpinned: the accumulation of bf16 reductions.  The oracle (like this
backend and torch) sums a bf16 row in fp32 and rounds once; the reference's
reduce keeps its accumulator in the input dtype
(nkipy/src/nkipy/core/ops/reduce.py:66-79), and no fixture says what its CPU
path returns for a bf16 np.sum (ml_dtypes is absent).  This reaches the row
sums of the Qwen3 softmax (decode and prefill).
"""
