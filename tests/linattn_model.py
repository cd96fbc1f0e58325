"""A CPU model of the fp16 operand path of the chunked linear-attention
kernel (nkipy_amd/csrc/kernels/linattn.hip), for tests: phi(x) = elu(x) + 1
evaluated in fp16 arithmetic, V, A / 256, S / 256 and z / 256 rounded to
fp16 (round to nearest even) as the kernel converts them, products of fp16
values accumulated in fp32 (float64 here, rounded once), the quotient in
fp32 and the output rounded to bf16.  It reproduces where the kernel's
operand window loses precision (values the fp16 conversions take into the
subnormal range), which the fp32 NumPy recurrence of the oracle does not.
It models the kernel; it is not a restatement of the reference.

``v_exp`` models a power-of-two prescale: V enters as fp16(v 2^v_exp), so
the state accumulates in those units and its copy stays fp16(S / 256); the
quotient is multiplied by 2^-v_exp (o is linear in v, so the prescale is
exact wherever it keeps the operands normal).
"""

from __future__ import annotations

import numpy as np

from oracle.numerics import bf16_round

F16 = np.float16


def phi_f16(x):
    """exp2(min(x, 0) * log2e) + max(x, 0) in fp16 arithmetic, x cast to fp16."""
    x = np.asarray(x, np.float32).astype(F16)
    t = (np.minimum(x, F16(0)) * F16(1.44269504088896340736)).astype(F16)
    e = np.exp2(t.astype(np.float32)).astype(F16)
    return (e + np.maximum(x, F16(0))).astype(F16)


def linear_attention_fp16(q, k, v, chunk=64, v_exp=0):
    """q, k, v (T, D) bf16 values of one sequence -> (T, D) bf16 values."""
    T, D = q.shape
    qf, kf = phi_f16(q).astype(np.float64), phi_f16(k).astype(np.float64)
    sv = float(2.0 ** v_exp)
    v16 = (np.asarray(v, np.float64) * sv).astype(np.float32).astype(F16).astype(np.float64)
    S = np.zeros((D, v.shape[1]), np.float32)
    z = np.zeros(D, np.float32)
    out = np.empty((T, v.shape[1]), np.float32)
    mask = np.tril(np.ones((chunk, chunk)))
    for c0 in range(0, T, chunk):
        Q, K, V = qf[c0:c0 + chunk], kf[c0:c0 + chunk], v16[c0:c0 + chunk]
        S16 = (S * np.float32(1 / 256)).astype(F16).astype(np.float64)
        z16 = (z * np.float32(1 / 256)).astype(F16).astype(np.float64)
        A = ((Q @ K.T).astype(np.float32) * mask).astype(np.float32)
        A16 = (A * np.float32(1 / 256)).astype(F16).astype(np.float64)
        num = (Q @ S16 + A16 @ V).astype(np.float32)
        den = (Q @ z16 + A16.sum(axis=1)).astype(np.float32)
        o = num * (np.float32(1) / den)[:, None]
        out[c0:c0 + chunk] = bf16_round(o * np.float32(1.0 / sv))
        S = (S + (K.T @ V).astype(np.float32)).astype(np.float32)
        z = (z + K.sum(axis=0)).astype(np.float32)
    return out
