"""The fp16 operand window of the linear-attention kernel, on the CPU: a
model of the kernel's operand path (tests/linattn_model.py) against the
oracle's fp32 recurrence over scales of v, the guard's decision on the
max |v| words the scan reports, and the lowering that wires the check."""

import numpy as np
import pytest
from linattn_model import linear_attention_fp16
from parity import record_close

from nkipy_amd.dispatch import launchers as LA
from oracle import kernels as K
from oracle.numerics import bf16_bits, bf16_round


def _inputs(T, sigma, seed=0):
    rng = np.random.default_rng(seed)
    q = bf16_round(rng.standard_normal((T, 128)) / np.sqrt(128))
    k = bf16_round(rng.standard_normal((T, 128)) / np.sqrt(128))
    v = bf16_round(rng.standard_normal((T, 128)) * sigma)
    return q, k, v


@pytest.mark.parametrize("sigma,ok", [(0.088, True), (1e-3, True), (1e-4, True), (3e-6, False)])
def test_model_of_the_fp16_path_has_a_small_v_edge(sigma, ok):
    """Within the bar down to v of std 1e-4; far outside it at 3e-6, where
    V and the state copy S / 256 are fp16 subnormals.  The guard's bound
    (max |v| >= 2^-13) sits between the two."""
    T = 1024
    q, k, v = _inputs(T, sigma)
    ref = K.linear_attention_chunked(q[None, None], k[None, None], v[None, None])[0, 0]
    ratio = record_close(linear_attention_fp16(q, k, v), ref, f"fp16 model, v std {sigma:g}", axis=-1)
    vmax = float(np.abs(v).max())
    if ok:
        assert ratio < 0.5 and vmax >= 2.0 ** -13
    else:
        assert ratio > 1.0 and vmax < 2.0 ** -13


def test_power_of_two_prescale_removes_the_edge():
    """o is linear in v: the same path on v 2^e (e putting max |v| in
    [8, 16)) and the output scaled back is within the bar at any scale."""
    T = 1024
    for sigma in (1e-5, 3e-6):
        q, k, v = _inputs(T, sigma, seed=1)
        ref = K.linear_attention_chunked(q[None, None], k[None, None], v[None, None])[0, 0]
        e = int(4 - np.ceil(np.log2(np.abs(v).max())))
        assert record_close(linear_attention_fp16(q, k, v, v_exp=e), ref, f"prescaled, v std {sigma:g}",
                            axis=-1) < 0.5


def test_guard_decision_on_reported_max_abs_v():
    bits = lambda x: bf16_bits(np.asarray(x, np.float32)).astype(np.uint32)
    LA.check_linear_attention_vmax(bits([0.3, 2.0 ** -13, 0.0, 60000.0]))  # in window, or all zero
    with pytest.raises(LA.LinearAttentionRangeError, match="below 2\\^-13"):
        LA.check_linear_attention_vmax(bits([0.3, 5e-5]))
    with pytest.raises(LA.LinearAttentionRangeError, match="65536"):
        LA.check_linear_attention_vmax(bits([65536.0, 0.3]))
    with pytest.raises(LA.LinearAttentionRangeError, match="non-finite"):
        LA.check_linear_attention_vmax(np.array([0x7F80], np.uint32))


def test_lowering_registers_the_window_check():
    from nkipy_amd.core import dtypes as dt
    from nkipy_amd.core.trace import NKIPyKernel
    from nkipy_amd.dispatch.lower import lower
    from nkipy_amd.kernels import chunked_linear_attention_kernel

    q = dt.to_bf16(np.zeros((2, 4, 1024, 128), np.float32))
    plan = lower(NKIPyKernel.trace(chunked_linear_attention_kernel).specialize(q, q, q))
    (chk,) = plan.checks
    assert chk["kind"] == "linattn_vmax" and chk["count"] == 8
    assert plan.buffers[chk["buffer"]].kind == "temp" and plan.buffers[chk["buffer"]].nbytes == 32
    ((*_, scan),) = [st.launches(lambda v: 1 << 40) for st in plan.steps]
    assert scan.args.vmax
