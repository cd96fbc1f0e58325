"""Benchmark of the hot path on one MI355X.

One JSON line on stdout.  Seven workloads run through the product path
(traced NumPy kernel -> plan -> gfx950 kernels through the C-ABI runtime),
each with its own roofline, CPU baseline and parity record:

  1  row softmax, x fp32 (2048, 4096)
  2  residual + RMSNorm, x, r bf16 (8192, 4096), w bf16 (4096,), eps 1e-6
     -- the headline: ``value`` is its achieved HBM bandwidth per step
  3  SwiGLU MLP, x (4096, 4096), W_gate / W_up (4096, 14336), W_down
     (14336, 4096), bf16
  4  chunked causal linear attention, q, k, v bf16 (4, 16, 8192, 128)
  5  Llama-style decoder layer with fp8 weights, x bf16 (8, 2048, 4096),
     32 / 8 heads, FFN 14336 -- reported as its latency per layer
  6  Qwen3 prefill attention: q bf16 (1, 2048, 32, 128) against a bf16 KV
     cache of 4096 rows (8 KV heads), scores rounded to bf16, mask rows
     [:2048, :4096], bf16 softmax (an extra line beside the five
     configurations)
  7  Qwen3 attention layer decode step: one token for each of 8 sequences
     (hidden 4096, 32 / 8 heads) against 4096-row bf16 caches at position
     4000 -- projections, q / k norm and RoPE, cache writes, attention,
     output projection (an extra line: the serving path)

Timing: inputs are resident in HBM; bandwidth-bound steps rotate over
buffer sets whose total exceeds the 256 MB Infinity Cache; every timed
region follows 50 ms of untimed load of the same work (the part ramps its
clocks) and is bracketed by HIP events on the runtime stream.  Per-kernel
times inside multi-kernel steps come from each launch run back to back with
itself over the rotating buffer sets (events around the whole run only, so
no marker sits between two launches of one kernel), after one whole step
has produced every intermediate.

``cpu_baseline`` of each workload is the oracle's NumPy form of the same
kernel (the reference's CPU path) timed on the host on a bounded sample;
the same leg checks the GPU output against it (``parity``).

Profiling: ``--mark-sections`` launches a marker copy kernel (grid 1000 +
workload id) before each workload, so a rocprofv3 kernel trace or counter
run of this script can be split per workload and per launch position;
``python bench.py --summarize DIR`` prints those summaries (no GPU needed).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                       [--configs 1,2,3,4,5,6,7] [--mark-sections] [--calibrate-copy]
       python bench.py --summarize DIR [--traffic-json PATH]
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0
MALL_BYTES = 256 * 2**20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
METRIC = "per-kernel achieved HBM GB/s & MFMA TFLOP/s vs peak; fp8 decoder-layer latency (us)"

# workload sizes
SM_ROWS, SM_N = 2048, 4096
RMS_ROWS, RMS_N, RMS_EPS = 8192, 4096, 1e-6
MLP_M, MLP_H, MLP_F = 4096, 4096, 14336
LA_B, LA_H, LA_T, LA_D = 4, 16, 8192, 128
DEC_B, DEC_S, DEC_HQ, DEC_HKV, DEC_D, DEC_F = 8, 2048, 32, 8, 128, 14336
DEC_HID = DEC_HQ * DEC_D
DEC_M = DEC_B * DEC_S
QP_B, QP_S, QP_MAXS, QP_HQ, QP_HKV = 1, 2048, 4096, 32, 8
# Qwen3 attention layer, one decode token per sequence
QD_B, QD_MAXS, QD_POS, QD_HID, QD_HQ, QD_HKV, QD_EPS = 8, 4096, 4000, 4096, 32, 8, 1e-6
QD_OTHER_BATCHES = (1, 32)


def _linattn_prefix_bytes():
    from nkipy_amd.dispatch.launchers import linear_attention_split

    _, rchunks, nranges = linear_attention_split(LA_B * LA_H, LA_T)
    return 2 * LA_B * LA_H * nranges * rchunks * 64 * LA_D * 2


# Per workload: (name, [(launch label, bound, algorithmic work per launch)])
# -- bytes for "hbm", flops for "mfma"; the launches of one step, in order.
def sections():
    norm_bytes = 2 * DEC_M * DEC_HID * 2 + DEC_HID * 2
    return {
        1: ("softmax", [("softmax", "hbm", SM_ROWS * SM_N * 4 * 2)]),
        2: ("residual_rmsnorm", [("residual_rmsnorm", "hbm", RMS_ROWS * RMS_N * 2 * 3 + RMS_N * 2)]),
        3: ("swiglu_mlp", [("gate_up_swiglu", "mfma", 2 * 2 * MLP_M * MLP_H * MLP_F),
                           ("down_proj", "mfma", 2 * MLP_M * MLP_F * MLP_H)]),
        4: ("linear_attention", [("prefix_states", "hbm", _linattn_prefix_bytes()),
                                 ("scan", "hbm", 4 * LA_B * LA_H * LA_T * LA_D * 2)]),
        5: ("decoder_layer_fp8", [
            ("attn_norm", "hbm", norm_bytes),
            # the QKV projection's epilogue also rotates q and k (RoPE)
            ("qkv_proj_rope", "mfma", 2 * DEC_M * DEC_HID * (DEC_HQ + 2 * DEC_HKV) * DEC_D),
            ("attention", "mfma", 4 * DEC_B * DEC_HQ * DEC_S * DEC_S * DEC_D // 2),
            ("o_proj_residual", "mfma", 2 * DEC_M * DEC_HID * DEC_HID),
            ("mlp_norm", "hbm", norm_bytes),
            ("gate_up_swiglu", "mfma", 2 * 2 * DEC_M * DEC_HID * DEC_F),
            ("down_proj_residual", "mfma", 2 * DEC_M * DEC_F * DEC_HID)]),
        # the bf16 softmax: row-max and row-sum passes over the scores (half
        # the flops each, recomputed by the last pass), then the weighted values
        6: ("qwen3_prefill_attention", [("rowmax", "mfma", 2 * QP_B * QP_HQ * QP_S * QP_S * DEC_D // 2),
                                        ("rowsum", "mfma", 2 * QP_B * QP_HQ * QP_S * QP_S * DEC_D // 2),
                                        ("attention", "mfma", 4 * QP_B * QP_HQ * QP_S * QP_S * DEC_D // 2)]),
        7: ("qwen3_decode_step", _decode_launches()),
        9: ("copy_calibration", [("copy16", "hbm", 2 * 2**30)]),
    }


def _decode_launches():
    """Bytes each launch of the Qwen3 decode step moves (its inputs and
    outputs as this decomposition has them: partial sums of the K-range
    projections, the fp32 scores and split outputs of the attention)."""
    from nkipy_amd.dispatch.launchers import gemv_mfma_preferred, gemv_mfma_split

    B, H, Hkv, D, hid = QD_B, QD_HQ, QD_HKV, DEC_D, QD_HID
    L, nqkv = QD_POS + 1, (QD_HQ + 2 * QD_HKV) * DEC_D
    nsp = -(-L // 128)
    assert gemv_mfma_preferred(B, nqkv, hid) and gemv_mfma_preferred(B, hid, H * D)
    ks1, _ = gemv_mfma_split(B, nqkv, hid)
    ks2, _ = gemv_mfma_split(B, hid, H * D)
    kv = 2 * B * L * Hkv * D
    return [("qkv_partials", "hbm", 2 * hid * nqkv + 2 * B * hid + 4 * ks1 * B * nqkv),
            # the q, k, v heads' partial sums in (added here); q out, k / v
            # into the caches' rows at pos
            ("head_rope_cache_rows", "hbm", 4 * ks1 * B * nqkv + 2 * B * (H + 2 * Hkv) * D),
            ("scores", "hbm", kv + 4 * B * H * L),
            ("rowstat", "hbm", 4 * B * H * L),
            ("values", "hbm", kv + 4 * B * H * L + 4 * B * H * nsp * D),
            ("combine", "hbm", 4 * B * H * nsp * D + 2 * B * H * D),
            ("o_partials", "hbm", 2 * H * D * hid + 2 * B * H * D + 4 * ks2 * B * hid),
            ("o_reduce", "hbm", 4 * ks2 * B * hid + 2 * B * hid)]


def _decode_step_bytes(B=QD_B):
    """Algorithmic HBM bytes of one decode step: both weights, the K / V
    rows attended, the token's activations and its cache rows."""
    H, Hkv, D, hid = QD_HQ, QD_HKV, DEC_D, QD_HID
    nqkv = (H + 2 * Hkv) * D
    return (2 * hid * nqkv + 2 * H * D * hid + 2 * 2 * B * (QD_POS + 1) * Hkv * D
            + 2 * 2 * B * hid + 2 * 2 * B * Hkv * D)


MARK_BASE = 1000  # marker grid = MARK_BASE + workload id
LAUNCH_MARK = 100  # marker grid = MARK_BASE + LAUNCH_MARK + launch index (back-to-back runs)
END_MARK = 99  # marker grid = MARK_BASE + END_MARK: the workload's labelled dispatches end
CUS, XCDS = 256, 8  # MI355X


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# seconds of untimed load before a timed region (clock ramp)
DEVICE_WARM_S = 0.05


def _sets_for(bytes_per_set: int) -> int:
    return max(2, math.ceil(3 * MALL_BYTES / bytes_per_set))


def _rate(bound, work, us):
    """(achieved, peak, unit) of ``work`` done in ``us`` microseconds."""
    if bound == "hbm":
        return work / (us * 1e-6) / 1e9, HBM_PEAK_GBS, "GB/s"
    return work / (us * 1e-6) / 1e12, BF16_PEAK_TFLOPS, "TFLOP/s"


class Marker:
    """Marker launches that split a profiler trace per workload."""

    def __init__(self, rt, enabled):
        self.rt, self.enabled = rt, enabled
        if enabled:
            self.n = 4096 * (MARK_BASE + LAUNCH_MARK + 64)
            self.src, self.dst = rt.malloc(self.n), rt.malloc(self.n)

    def mark(self, sid):
        if self.enabled:
            from nkipy_amd.dispatch.generic import copy16

            copy16(self.src, self.dst, 4096 * (MARK_BASE + sid)).run(self.rt)

    def mark_launch(self, i):
        """Before launch i of the current workload runs back to back with
        itself: every dispatch up to the next marker is that launch."""
        if self.enabled:
            self.mark(LAUNCH_MARK + i)

    def end(self):
        """Closes the current workload: dispatches up to the next workload
        marker are not labelled."""
        if self.enabled:
            self.mark(END_MARK)


def _time_steps(bounds, steps, warmup, rt, graph=False):
    """Mean milliseconds per step over ``steps`` steps run round robin over
    the bound plans, back to back on the runtime stream, bracketed by HIP
    events (event pairs around every launch would insert markers between
    kernels); ``graph`` replays each plan as its captured HIP graph."""
    run = (lambda b: b.run_graph()) if graph else (lambda b: b.run())
    for i in range(warmup):
        run(bounds[i % len(bounds)])
    rt.sync()
    # The part ramps its clocks over the first ~20 ms of sustained load, so
    # the timed region starts after DEVICE_WARM_S of the same work.
    t_end = time.perf_counter() + DEVICE_WARM_S
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(16):
            run(bounds[i % len(bounds)])
            i += 1
        rt.sync()
    e0, e1 = rt.event(), rt.event()
    e0.record()
    for k in range(steps):
        run(bounds[k % len(bounds)])
    e1.record()
    rt.sync()
    total = e0.elapsed_ms(e1)
    e0.destroy()
    e1.destroy()
    return total / steps


def _time_in_step(bounds, reps, rt, mk=None):
    """Mean microseconds of each launch of a step.  One whole step per buffer
    set first produces every intermediate; then launch i runs ``reps`` times
    back to back over the sets, with HIP events around that run only (an
    event between two launches adds a marker's latency to the shorter
    kernels).  A launch that writes over its own input reads its previous
    result: the kernels' work does not depend on the values."""
    n = len(bounds[0].launches)
    for b in bounds:
        b.run()
    rt.sync()
    out = []
    e0, e1 = rt.event(), rt.event()
    for i in range(n):
        if mk is not None:
            mk.mark_launch(i)
        for r in range(2):
            bounds[r % len(bounds)].run_range(i, i + 1)
        e0.record()
        for r in range(reps):
            bounds[r % len(bounds)].run_range(i, i + 1)
        e1.record()
        rt.sync()
        out.append(e0.elapsed_ms(e1) / reps * 1e3)
    e0.destroy()
    e1.destroy()
    return out


def _shape_of(launch):
    a = launch.args
    if hasattr(a, "K") and hasattr(a, "M"):
        return {"M": int(a.M), "N": int(a.N), "K": int(a.K)}
    return None


def _kernel_records(sid, launches, us_list):
    recs = []
    for (label, bound, work), l, us in zip(sections()[sid][1], launches, us_list):
        ach, peak, unit = _rate(bound, work, us)
        r = {"label": label, "kernel": l.symbol, "grid": l.grid[0], "us": round(us, 2),
             "bound": bound, "work": work, "achieved": round(ach, 1), "peak": peak, "unit": unit,
             "frac": round(ach / peak, 4)}
        sh = _shape_of(l)
        if sh:
            r["shape"] = sh
        recs.append(r)
    return recs


def _traffic(key):
    """HBM bytes per launch of ``key`` ("workload/label") from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (profiles/traffic.json)."""
    try:
        with open(TRAFFIC_FILE) as f:
            entry = json.load(f).get(key)
    except (OSError, ValueError):
        return None
    return entry.get("total_bytes") if isinstance(entry, dict) else None


def _roofline(sid, rec, us=None, work=None):
    """Roofline block of one kernel record (or of a whole step with ``us`` /
    ``work`` given)."""
    name = sections()[sid][0]
    bound = rec["bound"]
    us = rec["us"] if us is None else us
    work = rec["work"] if work is None else work
    ach, peak, unit = _rate(bound, work, us)
    return {"bound": bound, "kernel": rec["kernel"], "achieved": round(ach, 1), "peak": peak, "unit": unit,
            "frac": round(ach / peak, 4), "traffic": _traffic(f"{name}/{rec['label']}"),
            "work_per_launch": work, "us_per_launch": round(us, 3)}


# ---------------------------------------------------------------------------
# parity of a GPU output against the oracle (inside the cpu_baseline leg)
# ---------------------------------------------------------------------------
def _parity(got, ref, bar="bf16", atol=1e-2):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    out = {"n": int(err.size), "finite": bool(np.all(np.isfinite(got))), "max_abs": float(err.max()),
           "max_rel": float(np.max(err / np.maximum(np.abs(ref), 1e-30)))}
    if bar == "fp32":
        ratio = out["max_rel"] / 1e-5
        out["bar"] = "max |got - ref| / |ref| <= 1e-5"
    else:
        a = min(atol, 2e-2 * float(np.sqrt(np.mean(ref ** 2))))
        ratio = float(np.max(err / (2e-2 * np.abs(ref) + a)))
        out["bar"] = f"|got - ref| <= 2e-2 |ref| + {a:.3g}"
    out["worst_of_bar"] = round(ratio, 4)
    out["ok"] = bool(out["finite"] and ratio <= 1.0)
    return out


def _timed(fn, runs):
    fn_out = None
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn_out = fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), times, fn_out


def _blas_threads():
    try:
        from threadpoolctl import threadpool_info

        return max((p.get("num_threads", 1) for p in threadpool_info() if p.get("user_api") == "blas"), default=1)
    except Exception:  # pragma: no cover
        return None


def _host_cores():
    return len(os.sched_getaffinity(0))


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------
def bench_softmax(a, rt, mk):
    from nkipy_amd.kernels import softmax_kernel
    from nkipy_amd.runtime import DeviceKernel, DeviceTensor

    rng = np.random.default_rng(42)
    x = (rng.standard_normal((SM_ROWS, SM_N)) * 4).astype(np.float32)
    dk = DeviceKernel.compile_and_load(softmax_kernel, x, name="softmax")
    if dk.plan.kernel_kinds != ["softmax"]:
        raise RuntimeError(f"softmax did not lower to the fused kernel: {dk.plan.kernel_kinds}")
    work = sections()[1][1][0][2]
    sets = [(DeviceTensor.from_numpy(x, name="x"), DeviceTensor.empty((SM_ROWS, SM_N), np.float32, name="output0"))
            for _ in range(_sets_for(work))]
    bounds = [dk.executor.bind({"x": s[0].ptr, "output0": s[1].ptr}) for s in sets]
    mk.mark(1)
    ms = _time_steps(bounds, a.steps, a.warmup, rt)
    recs = _kernel_records(1, bounds[0].launches, [ms * 1e3])
    entry = {"config": 1, "workload": "softmax", "shape": [SM_ROWS, SM_N], "dtype": "f32",
             "us_per_step": round(ms * 1e3, 3), "roofline": _roofline(1, recs[0]), "kernels": recs,
             "buffer_sets": len(sets)}

    def cpu():
        from oracle import kernels as K

        t, ts, ref = _timed(lambda: K.softmax_kernel(x), 5)
        return ({"value": round(work / t / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                 "sample": f"full workload, median of {len(ts)} runs ({sum(ts):.2f} s); NumPy elementwise "
                           f"ops are single-threaded; host has {_host_cores()} cores",
                 "ms": round(t * 1e3, 2)},
                _parity(sets[0][1].numpy(), ref, bar="fp32"))

    return entry, cpu


def bench_rmsnorm(a, rt, mk):
    from nkipy_amd.core import dtypes as dt
    from nkipy_amd.kernels import residual_rmsnorm_kernel
    from nkipy_amd.runtime import DeviceKernel, DeviceTensor

    rng = np.random.default_rng(42)
    x = dt.round_to_bf16(rng.standard_normal((RMS_ROWS, RMS_N)).astype(np.float32))
    r = dt.round_to_bf16(rng.standard_normal((RMS_ROWS, RMS_N)).astype(np.float32))
    w = dt.round_to_bf16(rng.uniform(0.5, 1.5, RMS_N).astype(np.float32))
    xb, rb, wb = dt.to_bf16(x), dt.to_bf16(r), dt.to_bf16(w)
    dk = DeviceKernel.compile_and_load(residual_rmsnorm_kernel, xb, rb, wb, RMS_EPS, name="residual_rmsnorm")
    if dk.plan.kernel_kinds != ["rmsnorm"]:
        raise RuntimeError(f"residual rmsnorm did not lower to the fused kernel: {dk.plan.kernel_kinds}")
    work = sections()[2][1][0][2]
    wt = DeviceTensor.from_numpy(wb, name="weight")
    sets = [(DeviceTensor.from_numpy(xb, name="x"), DeviceTensor.from_numpy(rb, name="residual"),
             DeviceTensor.empty((RMS_ROWS, RMS_N), dt.bfloat16, name="output0")) for _ in range(_sets_for(work))]
    bounds = [dk.executor.bind({"x": s[0].ptr, "residual": s[1].ptr, "weight": wt.ptr, "output0": s[2].ptr})
              for s in sets]
    mk.mark(2)
    ms = _time_steps(bounds, a.steps, a.warmup, rt)
    recs = _kernel_records(2, bounds[0].launches, [ms * 1e3])
    entry = {"config": 2, "workload": "residual_rmsnorm", "shape": [RMS_ROWS, RMS_N], "dtype": "bf16",
             "eps": RMS_EPS, "us_per_step": round(ms * 1e3, 3), "ms_per_step": ms,
             "roofline": _roofline(2, recs[0]), "kernels": recs, "buffer_sets": len(sets)}

    def cpu():
        from oracle import kernels as K

        K.residual_rmsnorm_bf16(x[:64], r[:64], w, RMS_EPS)
        t, ts, ref = _timed(lambda: K.residual_rmsnorm_bf16(x, r, w, RMS_EPS), 5)
        return ({"value": round(work / t / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                 "sample": f"full workload (bf16 values held in fp32 arrays), median of {len(ts)} runs "
                           f"({sum(ts):.2f} s); NumPy elementwise ops are single-threaded; "
                           f"host has {_host_cores()} cores",
                 "ms": round(t * 1e3, 2)},
                _parity(dt.to_float32(sets[0][2].numpy()), ref))

    return entry, cpu


def bench_swiglu(a, rt, mk):
    from nkipy_amd.core import dtypes as dt
    from nkipy_amd.kernels import swiglu_mlp_kernel
    from nkipy_amd.runtime import DeviceKernel, DeviceTensor

    rng = np.random.default_rng(42)
    x = dt.round_to_bf16(rng.standard_normal((MLP_M, MLP_H)).astype(np.float32))
    ws = [dt.round_to_bf16((rng.standard_normal(s) * 0.02).astype(np.float32))
          for s in ((MLP_H, MLP_F), (MLP_H, MLP_F), (MLP_F, MLP_H))]
    args = [dt.to_bf16(v) for v in [x] + ws]
    dk = DeviceKernel.compile_and_load(swiglu_mlp_kernel, *args, name="swiglu_mlp")
    if dk.plan.kernel_kinds != ["gemm_swiglu", "gemm"]:
        raise RuntimeError(f"SwiGLU did not lower to the fused GEMMs: {dk.plan.kernel_kinds}")
    ins = {n: DeviceTensor.from_numpy(v, name=n) for n, v in zip(("x", "w_gate", "w_up", "w_down"), args)}
    out = DeviceTensor.empty((MLP_M, MLP_H), dt.bfloat16, name="output0")
    bound = dk.executor.bind({**{k: v.ptr for k, v in ins.items()}, "output0": out.ptr})
    steps, warm = max(5, a.steps // 20), max(2, a.warmup // 5)
    mk.mark(3)
    ms = _time_steps([bound], steps, warm, rt)
    recs = _kernel_records(3, bound.launches, _time_in_step([bound], max(3, steps), rt, mk))
    flops = sum(w for _, _, w in sections()[3][1])
    step_rec = {"label": "mlp", "kernel": " + ".join(l.symbol for l in bound.launches), "bound": "mfma"}
    entry = {"config": 3, "workload": "swiglu_mlp", "shape": {"M": MLP_M, "hidden": MLP_H, "ffn": MLP_F},
             "dtype": "bf16", "us_per_step": round(ms * 1e3, 2),
             "roofline": _roofline(3, step_rec, us=ms * 1e3, work=flops), "kernels": recs}

    def cpu():
        from oracle import kernels as K
        from oracle import numerics as N

        rows = np.arange(0, MLP_M, 16)  # 256 rows: rows are independent
        K.swiglu_mlp(x[:8], *ws)
        t, ts, ref = _timed(lambda: K.swiglu_mlp(x[rows], *ws, round_h=N.bf16_round), 3)
        f = flops * len(rows) / MLP_M
        return ({"value": round(f / t / 1e12, 3), "unit": "TFLOP/s", "cores": _blas_threads(),
                 "kind": "port", "blas_threads": _blas_threads(),
                 "sample": f"{len(rows)} of {MLP_M} rows (fp32 NumPy matmuls on OpenBLAS), median of "
                           f"{len(ts)} runs ({sum(ts):.2f} s); host has {_host_cores()} cores",
                 "ms_full_equiv": round(t * MLP_M / len(rows) * 1e3, 1)},
                _parity(dt.to_float32(out.numpy()[rows]), ref))

    return entry, cpu


def bench_linattn(a, rt, mk):
    from nkipy_amd.core import dtypes as dt
    from nkipy_amd.kernels import chunked_linear_attention_kernel
    from nkipy_amd.runtime import DeviceKernel, DeviceTensor

    shape = (LA_B, LA_H, LA_T, LA_D)
    rng = np.random.default_rng(42)
    host = [dt.round_to_bf16((rng.standard_normal(shape) / np.sqrt(LA_D)).astype(np.float32)) for _ in range(3)]
    args = [dt.to_bf16(v) for v in host]
    dk = DeviceKernel.compile_and_load(chunked_linear_attention_kernel, *args, name="linear_attention")
    if dk.plan.kernel_kinds != ["linear_attention"]:
        raise RuntimeError(f"linear attention did not lower to the fused kernel: {dk.plan.kernel_kinds}")
    work = 4 * LA_B * LA_H * LA_T * LA_D * 2
    sets = [[DeviceTensor.from_numpy(v, name=nm) for nm, v in zip("qkv", args)]
            + [DeviceTensor.empty(shape, dt.bfloat16, name="output0")] for _ in range(_sets_for(work))]
    bounds = [dk.executor.bind({"q": s[0].ptr, "k": s[1].ptr, "v": s[2].ptr, "output0": s[3].ptr}) for s in sets]
    if len(bounds[0].launches) != len(sections()[4][1]):
        raise RuntimeError("linear attention step has an unexpected launch count")
    steps, warm = max(10, a.steps // 10), max(2, a.warmup // 5)
    mk.mark(4)
    ms = _time_steps(bounds, steps, warm, rt)
    recs = _kernel_records(4, bounds[0].launches, _time_in_step(bounds, max(5, steps), rt, mk))
    step_rec = {"label": "step", "kernel": " + ".join(l.symbol for l in bounds[0].launches), "bound": "hbm"}
    roof = _roofline(4, step_rec, us=ms * 1e3, work=work)
    t_pre, t_scan = _traffic("linear_attention/prefix_states"), _traffic("linear_attention/scan")
    roof["traffic"] = (t_pre + t_scan) if (t_pre and t_scan) else None
    entry = {"config": 4, "workload": "chunked_linear_attention", "shape": list(shape), "chunk": 64,
             "dtype": "bf16", "us_per_step": round(ms * 1e3, 2), "roofline": roof, "kernels": recs,
             "flops_per_step": sum(l.flops for l in bounds[0].launches), "buffer_sets": len(sets)}

    def cpu():
        from oracle import kernels as K

        heads = [(0, 0), (3, 15)]
        sample = lambda: [K.linear_attention_chunked(*[v[b:b + 1, h:h + 1] for v in host]) for b, h in heads]
        t, ts, refs = _timed(sample, 3)
        per_head = 4 * LA_T * LA_D * 2
        got = dt.to_float32(sets[0][3].numpy())
        return ({"value": round(per_head * len(heads) / t / 1e9, 3), "unit": "GB/s", "cores": _blas_threads(),
                 "kind": "port", "blas_threads": _blas_threads(),
                 "sample": f"{len(heads)} of {LA_B * LA_H} heads (fp32 chunked recurrence in NumPy), median "
                           f"of {len(ts)} runs ({sum(ts):.2f} s); host has {_host_cores()} cores",
                 "ms_full_equiv": round(t * LA_B * LA_H / len(heads) * 1e3, 1)},
                _parity(np.concatenate([got[b:b + 1, h:h + 1] for b, h in heads]), np.concatenate(refs)))

    return entry, cpu


def _quantize_fp8(rng, shape):
    """N(0, 0.02) weights -> e4m3fn codes, per-output-channel scale amax / 448."""
    import torch

    w = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02))
    scale = (w.abs().amax(dim=1) / 448.0).clamp_min(1e-12)
    codes = (w / scale[:, None]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return codes, scale.numpy().astype(np.float32)


def bench_decoder(a, rt, mk):
    from nkipy_amd.core import dtypes as dt
    from nkipy_amd.kernels import llama_decoder_layer_fp8
    from nkipy_amd.runtime import DeviceKernel, DeviceTensor

    B, S, hid = DEC_B, DEC_S, DEC_HID
    rng = np.random.default_rng(42)
    x = dt.round_to_bf16(rng.standard_normal((B, S, hid), dtype=np.float32))
    w = {"n_heads": DEC_HQ, "n_kv_heads": DEC_HKV, "eps": 1e-5, "rope_theta": 5.0e5,
         "attn_norm": np.ones(hid, np.float32), "mlp_norm": np.ones(hid, np.float32)}
    for name, shp in (("wqkv", ((DEC_HQ + 2 * DEC_HKV) * DEC_D, hid)), ("wo", (hid, hid)),
                      ("w_gate", (DEC_F, hid)), ("w_up", (DEC_F, hid)), ("w_down", (hid, DEC_F))):
        w[name], w[name + "_scale"] = _quantize_fp8(rng, shp)
    f8 = lambda c: c.view(dt.float8_e4m3fn)
    args = [dt.to_bf16(x), dt.to_bf16(w["attn_norm"]), f8(w["wqkv"]), w["wqkv_scale"], f8(w["wo"]),
            w["wo_scale"], dt.to_bf16(w["mlp_norm"]), f8(w["w_gate"]), w["w_gate_scale"], f8(w["w_up"]),
            w["w_up_scale"], f8(w["w_down"]), w["w_down_scale"]]
    dk = DeviceKernel.compile_and_load(llama_decoder_layer_fp8, *args, name="decoder_layer_fp8")
    kinds = ["rmsnorm", "gemm_rope", "attention", "gemm", "rmsnorm", "gemm_swiglu", "gemm"]
    if dk.plan.kernel_kinds != kinds:
        raise RuntimeError(f"decoder layer did not lower to the fused kernels: {dk.plan.kernel_kinds}")
    names = [p.name for p in dk.graph.parameters]
    ins = {n: DeviceTensor.from_numpy(v, name=n) for n, v in zip(names, args)}
    # the activations rotate over three sets (384 MB), so the first RMSNorm
    # reads x from HBM, and each set has its own executor, i.e. its own
    # intermediates (the second RMSNorm's input, the projections' outputs),
    # so that a launch run back to back over the sets reads them from HBM
    # too; the weights stay as they are
    from nkipy_amd.dispatch.plan import PlanExecutor

    xs = [ins[names[0]]] + [DeviceTensor.from_numpy(args[0], name=names[0]) for _ in range(2)]
    outs = [DeviceTensor.empty((B, S, hid), dt.bfloat16, name="output0") for _ in xs]
    exs = [dk.executor] + [PlanExecutor(dk.plan, lower_fn=dk.executor.lower_fn) for _ in xs[1:]]
    bounds = [ex.bind({**{k: v.ptr for k, v in ins.items()}, names[0]: xv.ptr, "output0": o.ptr})
              for ex, xv, o in zip(exs, xs, outs)]
    steps, warm = max(5, a.steps // 20), max(2, a.warmup // 5)
    mk.mark(5)
    ms = _time_steps(bounds, steps, warm, rt)
    recs = _kernel_records(5, bounds[0].launches, _time_in_step(bounds, max(6, steps), rt, mk))
    flops = sum(l.flops for l in bounds[0].launches)
    ach = flops / (ms * 1e-3) / 1e12
    roof = {"bound": "mfma", "kernel": "layer (9 kernels)", "achieved": round(ach, 1), "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(ach / BF16_PEAK_TFLOPS, 4),
            "frac_of_fp8_peak": round(ach / FP8_PEAK_TFLOPS, 4), "traffic": None,
            "work_per_launch": flops, "us_per_launch": round(ms * 1e3, 1),
            "note": "fp8 weights are decoded exactly to bf16 for bf16 MFMAs (the activations stay bf16), "
                    "so the bf16 dense peak is the ceiling; the fp8 fraction is given for reference"}
    entry = {"config": 5, "workload": "llama_decoder_layer_fp8",
             "shape": {"batch": B, "seq": S, "hidden": hid, "heads": DEC_HQ, "kv_heads": DEC_HKV,
                       "head_dim": DEC_D, "ffn": DEC_F},
             "dtype": "bf16 activations, e4m3fn weights with per-channel fp32 scales",
             "value": round(ms * 1e3, 1), "unit": "us per layer", "higher_is_better": False,
             "us_per_step": round(ms * 1e3, 1), "flops_per_layer": flops, "roofline": roof, "kernels": recs}

    def cpu():
        from oracle import kernels as K

        t0 = time.perf_counter()
        ref = K.decoder_layer_fp8(x[0:1], w)["y"]
        t = time.perf_counter() - t0
        f = flops / B
        return ({"value": round(t * B * 1e6, 0), "unit": "us per layer (scaled from one sequence)",
                 "tflops": round(f / t / 1e12, 3), "cores": _blas_threads(), "kind": "port",
                 "blas_threads": _blas_threads(),
                 "sample": f"1 of {B} sequences ({S} tokens, fp32 NumPy with OpenBLAS matmuls, weights "
                           f"dequantized per call like the NumPy kernel), one run ({t:.2f} s); host has "
                           f"{_host_cores()} cores"},
                _decoder_parity(dt.to_float32(outs[0].numpy()[0:1]), ref))

    return entry, cpu


def _decoder_parity(got, ref):
    """End to end through eight bf16 cast points: the floor 2e-2 x RMS, and
    (recorded beside it) the reference's absolute tolerance 1e-2
    (tests/utils.py:19-25) with the bf16 rtol 2e-2."""
    par = _parity(got, ref, atol=np.inf)
    tight = _parity(got, ref, atol=1e-2)
    par["atol_1e-2"] = {"bar": tight["bar"], "worst_of_bar": tight["worst_of_bar"], "ok": tight["ok"]}
    return par


def bench_qwen3_prefill(a, rt, mk):
    from nkipy_amd.core import dtypes as dt
    from nkipy_amd.kernels.qwen3 import prefill_attention_kernel
    from nkipy_amd.runtime import DeviceKernel, DeviceTensor

    B, S, MAXS, Hq, Hkv, D = QP_B, QP_S, QP_MAXS, QP_HQ, QP_HKV, DEC_D
    rng = np.random.default_rng(42)
    q = dt.round_to_bf16(rng.standard_normal((B, S, Hq, D), dtype=np.float32))
    ck = dt.round_to_bf16(rng.standard_normal((B, MAXS, Hkv, D), dtype=np.float32))
    cv = dt.round_to_bf16(rng.standard_normal((B, MAXS, Hkv, D), dtype=np.float32))
    args = [dt.to_bf16(v) for v in (q, ck, cv)]
    dk = DeviceKernel.compile_and_load(prefill_attention_kernel, *args, name="qwen3_prefill_attention")
    if dk.plan.kernel_kinds != ["attention"]:
        raise RuntimeError(f"Qwen3 prefill attention did not lower to one kernel: {dk.plan.kernel_kinds}")
    names = list(dk.input_tensors_info)
    sets = [[DeviceTensor.from_numpy(v, name=n) for n, v in zip(names, args)]
            + [DeviceTensor.empty((B, S, Hq, D), dt.bfloat16, name="output0")] for _ in range(3)]
    bounds = [dk.executor.bind({**{n: t.ptr for n, t in zip(names, s[:3])}, "output0": s[3].ptr}) for s in sets]
    if len(bounds[0].launches) != len(sections()[6][1]):
        raise RuntimeError("Qwen3 prefill attention step has an unexpected launch count")
    steps, warm = max(10, a.steps // 10), max(2, a.warmup // 5)
    mk.mark(6)
    ms = _time_steps(bounds, steps, warm, rt)
    recs = _kernel_records(6, bounds[0].launches, _time_in_step(bounds, max(5, steps), rt, mk))
    # the roofline of the whole step on the algorithmic (causal) flops: the
    # score products of the row-max and row-sum passes are recomputed work,
    # not counted
    step_rec = {"label": "step", "kernel": " + ".join(l.symbol for l in bounds[0].launches), "bound": "mfma"}
    roof = _roofline(6, step_rec, us=ms * 1e3, work=sections()[6][1][2][2])
    tr = [_traffic(f"qwen3_prefill_attention/{lbl}") for lbl, _, _ in sections()[6][1]]
    roof["traffic"] = sum(tr) if all(tr) else None
    entry = {"config": 6, "workload": "qwen3_prefill_attention",
             "shape": {"batch": B, "seq": S, "cache_rows": MAXS, "heads": Hq, "kv_heads": Hkv, "head_dim": D},
             "dtype": "bf16 (scores rounded to bf16 after the product and the divide by sqrt(d); "
                      "bf16 softmax)",
             "us_per_step": round(ms * 1e3, 2), "roofline": roof, "kernels": recs,
             "note": "causal flops (keys 0..s for query s); cache rows past S are masked and not read"}

    def cpu():
        from oracle import kernels as K

        rows = np.arange(0, S, 64)  # 32 query rows, across the causal range
        K.qwen3_prefill_attention(q, ck, cv, rows=rows[:1])
        t, ts, ref = _timed(lambda: K.qwen3_prefill_attention(q, ck, cv, rows=rows), 3)
        f = sum(4 * Hq * (int(r) + 1) * D for r in rows) * B
        got = dt.to_float32(sets[0][3].numpy())[:, rows]
        par = _parity(got, ref)
        rms = np.sqrt(np.mean(np.asarray(ref, np.float64) ** 2, axis=-1, keepdims=True))
        par["worst_of_bar_per_row_rms"] = round(float(np.max(
            np.abs(got - ref) / (2e-2 * np.abs(ref) + np.minimum(1e-2, 2e-2 * rms)))), 4)
        return ({"value": round(f / t / 1e12, 4), "unit": "TFLOP/s", "cores": 1, "kind": "port",
                 "sample": f"{len(rows)} of {S} query rows, all heads (NumPy op-by-op bf16 emulation over "
                           f"the {MAXS}-row cache), median of {len(ts)} runs ({sum(ts):.2f} s); host has "
                           f"{_host_cores()} cores",
                 "ms_full_equiv": round(t * S / len(rows) * 1e3, 1)}, par)

    return entry, cpu


def _decode_case(B, rt):
    """The traced Qwen3 decode layer at batch B with its rotating buffer
    sets: (kernel, sets of (inputs, outputs), bound plans, host arrays)."""
    from nkipy_amd.core import dtypes as dt
    from nkipy_amd.kernels.qwen3 import qwen3_attention_kernel
    from nkipy_amd.runtime import DeviceKernel, DeviceTensor

    MAXS, pos, hid, H, Hkv, D = QD_MAXS, QD_POS, QD_HID, QD_HQ, QD_HKV, DEC_D

    def decode(x, qkv_weight, q_norm_weight, k_norm_weight, cache_k, cache_v, start_pos, o_weight):
        return qwen3_attention_kernel(x, qkv_weight, q_norm_weight, k_norm_weight, QD_EPS, H, D, Hkv,
                                      cache_k, cache_v, start_pos, o_weight)

    rng = np.random.default_rng(42 + B)
    host = {"x": dt.round_to_bf16(rng.standard_normal((B, 1, hid), dtype=np.float32)),
            "qkv_weight": dt.round_to_bf16(rng.standard_normal((hid, (H + 2 * Hkv) * D), dtype=np.float32)
                                           * hid ** -0.5),
            "q_norm_weight": dt.round_to_bf16(rng.uniform(0.5, 1.5, D).astype(np.float32)),
            "k_norm_weight": dt.round_to_bf16(rng.uniform(0.5, 1.5, D).astype(np.float32)),
            "cache_k": dt.round_to_bf16(rng.standard_normal((B, MAXS, Hkv, D), dtype=np.float32)),
            "cache_v": dt.round_to_bf16(rng.standard_normal((B, MAXS, Hkv, D), dtype=np.float32)),
            "o_weight": dt.round_to_bf16(rng.standard_normal((H * D, hid), dtype=np.float32) * (H * D) ** -0.5)}
    order = ["x", "qkv_weight", "q_norm_weight", "k_norm_weight", "cache_k", "cache_v"]
    args = [dt.to_bf16(host[n]) for n in order] + [np.array([pos], np.int32), dt.to_bf16(host["o_weight"])]
    dk = DeviceKernel.compile_and_load(decode, *args, name=f"qwen3_decode_step_b{B}")
    names = [p.name for p in dk.graph.parameters]
    # every set holds its own weights and caches: a layer's weights are not
    # cache-resident between its steps in a model of many layers
    sets = []
    for _ in range(_sets_for(sum(v.nbytes for v in args))):
        ins = {n: DeviceTensor.from_numpy(v, name=n) for n, v in zip(names, args)}
        outs = {"output0": DeviceTensor.empty((B, 1, hid), dt.bfloat16, name="output0"),
                "cache_k": ins["cache_k.must_alias_input"], "cache_v": ins["cache_v.must_alias_input"]}
        sets.append((ins, outs))
    bounds = [dk.executor.bind(dk._io_ptrs(i, o)) for i, o in sets]
    return dk, sets, bounds, host


def _sync_call_us(dk, ins, outs, n=50, graph=False):
    """One synchronous call at a time (host dispatch, launches, wait): the
    latency a serving loop that waits for each token sees; ``graph`` replays
    the step as one captured HIP graph."""
    for _ in range(10):
        dk(ins, outs, graph=graph)
    t0 = time.perf_counter()
    for _ in range(n):
        dk(ins, outs, graph=graph)
    return (time.perf_counter() - t0) / n * 1e6


def bench_qwen3_decode(a, rt, mk):
    from nkipy_amd.core import dtypes as dt

    B, MAXS, pos, hid, H, Hkv, D = QD_B, QD_MAXS, QD_POS, QD_HID, QD_HQ, QD_HKV, DEC_D
    steps, warm = max(20, a.steps // 2), max(5, a.warmup)
    dk, sets, bounds, host = _decode_case(B, rt)
    if len(bounds[0].launches) != len(sections()[7][1]):
        raise RuntimeError(f"Qwen3 decode step has an unexpected launch list: "
                           f"{[l.symbol for l in bounds[0].launches]}")
    mk.mark(7)
    ms = _time_steps(bounds, steps, warm, rt)
    recs = _kernel_records(7, bounds[0].launches, _time_in_step(bounds, max(20, steps // 2), rt, mk))
    mk.end()  # the synchronous calls and the other batch sizes below are not labelled
    ins0, outs0 = sets[0]
    sync_us = _sync_call_us(dk, ins0, outs0)
    # the same wait around the bound launch list alone (no argument handling)
    for _ in range(10):
        bounds[0].run()
        rt.sync()
    t0 = time.perf_counter()
    for _ in range(50):
        bounds[0].run()
        rt.sync()
    sync_bound_us = (time.perf_counter() - t0) / 50 * 1e6
    sync_graph_us = _sync_call_us(dk, ins0, outs0, graph=True)
    graph_ms = _time_steps(bounds, steps, warm, rt, graph=True)
    step_rec = {"label": "step", "kernel": " + ".join(l.symbol for l in bounds[0].launches), "bound": "hbm"}
    roof = _roofline(7, step_rec, us=ms * 1e3, work=_decode_step_bytes(B))
    roof["traffic"] = None
    # the same step at one token and at a larger batch (no per-launch split)
    batches = []
    for b in QD_OTHER_BATCHES:
        dkb, setsb, boundsb, _ = _decode_case(b, rt)
        msb = _time_steps(boundsb, steps, warm, rt)
        wb = _decode_step_bytes(b)
        batches.append({"batch": b, "us_per_step": round(msb * 1e3, 2),
                        "synchronous_call_us": round(_sync_call_us(dkb, *setsb[0]), 1),
                        "synchronous_graph_call_us": round(_sync_call_us(dkb, *setsb[0], graph=True), 1),
                        "launches": len(boundsb[0].launches), "bytes": wb,
                        "achieved_GBs": round(wb / (msb * 1e-3) / 1e9, 1),
                        "frac": round(wb / (msb * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
        del dkb, setsb, boundsb
    entry = {"config": 7, "workload": "qwen3_decode_step",
             "shape": {"batch": B, "cache_rows": MAXS, "position": pos, "hidden": hid, "heads": H,
                       "kv_heads": Hkv, "head_dim": D},
             "dtype": "bf16 (the traced cast points of the Qwen3 attention layer)",
             "us_per_step": round(ms * 1e3, 2), "synchronous_call_us": round(sync_us, 1),
             "synchronous_bound_launch_us": round(sync_bound_us, 1),
             "us_per_step_graph": round(graph_ms * 1e3, 2), "synchronous_graph_call_us": round(sync_graph_us, 1),
             "roofline": roof, "kernels": recs, "other_batches": batches,
             "note": "one token per sequence through the whole attention layer (QKV projection, q / k norm and "
                     "RoPE, cache writes, attention over pos + 1 cached rows, output projection); steps queued "
                     "back to back over rotating weight / cache sets; synchronous_call_us waits for each step; the "
                     "_graph figures replay each step as one captured HIP graph"}

    def cpu():
        from oracle import kernels as K

        f32 = {k: dt.to_float32(dt.to_bf16(v)) for k, v in host.items()}
        run = lambda: K.qwen3_decode_layer(f32["x"], f32["qkv_weight"], f32["q_norm_weight"], f32["k_norm_weight"],
                                           QD_EPS, H, Hkv, D, f32["cache_k"], f32["cache_v"], pos,
                                           f32["o_weight"])
        t, ts, ref = _timed(run, 3)
        got = dt.to_float32(outs0["output0"].numpy())
        return ({"value": round(t * 1e6, 0), "unit": "us per decode step", "cores": _blas_threads(),
                 "kind": "port",
                 "sample": f"the whole step, all {B} sequences (NumPy float64 products, op-by-op bf16 cast "
                           f"points), median of {len(ts)} runs; host has {_host_cores()} cores"},
                _parity(got, ref[0]))

    return entry, cpu


def calibrate_copy(rt, mk, nbytes=1 << 30, reps=3):
    """Plain streaming copy of a known size: rocprof's FETCH_SIZE / WRITE_SIZE
    for nk_copy16 read against 1 GiB give the counter scale factors."""
    from nkipy_amd.dispatch.generic import copy16

    src, dst = rt.malloc(nbytes), rt.malloc(nbytes)
    rt.memset(src, 0x5a, nbytes)
    mk.mark(9)
    l = copy16(src, dst, nbytes)
    for _ in range(reps):
        l.run(rt)
    rt.sync()
    rt.free(src)
    rt.free(dst)
    log(f"copy calibration: {reps} x nk_copy16 of {nbytes} bytes")


# ---------------------------------------------------------------------------
# profiler summaries (no GPU)
# ---------------------------------------------------------------------------
def _label_dispatches(rows):
    """rows: dicts with name, wgs (workgroups), dispatch, sorted by dispatch.
    Yields (workload id, launch label, row) for the launches of the marked
    sections: a marker (nk_copy16 with MARK_BASE + id workgroups) opens a
    section, whose launches are whole steps, labelled by position; a launch
    marker (MARK_BASE + LAUNCH_MARK + i) within it is followed by launch i
    run back to back with itself."""
    secs = sections()
    cur, pos, fixed = None, 0, None
    for r in rows:
        if r["name"].startswith("__amd"):
            continue  # runtime copies and fills
        if r["name"] == "nk_copy16" and (r["wgs"] - MARK_BASE) in secs:
            cur, pos, fixed = r["wgs"] - MARK_BASE, 0, None
            continue
        if r["name"] == "nk_copy16" and r["wgs"] - MARK_BASE == END_MARK:
            cur, pos, fixed = None, 0, None
            continue
        if r["name"] == "nk_copy16" and cur is not None and 0 <= r["wgs"] - MARK_BASE - LAUNCH_MARK < 64:
            fixed = r["wgs"] - MARK_BASE - LAUNCH_MARK
            continue
        if cur is None:
            continue
        labels = secs[cur][1]
        if fixed is not None:
            yield cur, labels[fixed][0], r
            continue
        yield cur, labels[pos % len(labels)][0], r
        pos += 1


def _order(secs):
    return lambda kv: (kv[0][0], [l for l, _, _ in secs[kv[0][0]][1]].index(kv[0][1]))


def summarize(d, traffic_json=None):
    secs = sections()
    out = []
    for path in sorted(glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)):
        rows = []
        for r in csv.DictReader(open(path)):
            rows.append({"name": r["Kernel_Name"],
                         "wgs": int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"])),
                         "dispatch": int(r["Dispatch_Id"]),
                         "us": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3})
        rows.sort(key=lambda r: r["dispatch"])
        agg = {}
        for sid, label, r in _label_dispatches(rows):
            agg.setdefault((sid, label), []).append(r)
        out.append(f"kernel trace: {os.path.relpath(path, d)}")
        out.append(f"{'workload/launch':<38} {'kernel':<34} {'wgs':>6} {'calls':>6} {'avg_us':>9} "
                   f"{'min_us':>9} {'max_us':>9} {'achieved':>10} {'frac':>7}")
        for (sid, label), rs in sorted(agg.items(), key=_order(secs)):
            us = [r["us"] for r in rs]
            avg = sum(us) / len(us)
            bound, work = {l: (b, w) for l, b, w in secs[sid][1]}[label]
            ach, peak, unit = _rate(bound, work, avg)
            out.append(f"{secs[sid][0] + '/' + label:<38} {rs[0]['name'][:34]:<34} {rs[0]['wgs']:>6} "
                       f"{len(us):>6} {avg:>9.2f} {min(us):>9.2f} {max(us):>9.2f} {ach:>8.1f} {unit[:2]} {ach / peak:>7.3f}")
        out.append("")
    traffic = {}
    for path in sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)):
        disp = {}
        for r in csv.DictReader(open(path)):
            k = int(r["Dispatch_Id"])
            e = disp.setdefault(k, {"name": r["Kernel_Name"],
                                    "wgs": int(r["Grid_Size"]) // max(1, int(r["Workgroup_Size"])),
                                    "dispatch": k, "c": {}})
            e["c"][r["Counter_Name"]] = e["c"].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        rows = sorted(disp.values(), key=lambda r: r["dispatch"])
        agg = {}
        for sid, label, r in _label_dispatches(rows):
            agg.setdefault((sid, label), []).append(r)
        names = sorted({c for r in rows for c in r["c"]})
        out.append(f"counters: {os.path.relpath(path, d)} ({', '.join(names)}; per dispatch, mean)")
        cal = agg.get((9, "copy16"))
        scale = {}
        if cal:
            for c, alg in (("FETCH_SIZE", 2**30), ("WRITE_SIZE", 2**30)):
                v = [r["c"][c] for r in cal if c in r["c"]]
                if v:
                    scale[c] = (sum(v) / len(v)) * 1024 / alg
                    out.append(f"calibration: nk_copy16 of 1 GiB each way reads {c} = {sum(v) / len(v):.1f} KiB "
                               f"(scale {scale[c]:.4f})")
        for (sid, label), rs in sorted(agg.items(), key=_order(secs)):
            if sid == 9:
                continue
            mean = {c: sum(r["c"].get(c, 0.0) for r in rs) / len(rs) for c in names}
            parts = [f"{secs[sid][0] + '/' + label:<38}", f"n={len(rs):<4}"]
            # GRBM_GUI_ACTIVE is summed over the 8 XCDs (each has its own
            # GRBM), SQ_VALU_MFMA_BUSY_CYCLES over the 1024 SIMDs and
            # SQ_BUSY_CU_CYCLES over the 256 CUs
            gui = mean.get("GRBM_GUI_ACTIVE", 0.0) / XCDS
            if "SQ_VALU_MFMA_BUSY_CYCLES" in mean and gui:
                parts.append(f"mfma_busy={mean['SQ_VALU_MFMA_BUSY_CYCLES'] / (4 * CUS * gui):.3f}")
            if "SQ_BUSY_CU_CYCLES" in mean and gui:
                parts.append(f"cu_busy={mean['SQ_BUSY_CU_CYCLES'] / (CUS * gui):.3f}")
            # wave-state counters as fractions of the waves' lifetime
            # (SQ_WAVE_CYCLES, same units): where the waves spend their time
            if mean.get("SQ_WAVE_CYCLES"):
                for c in names:
                    if c.startswith(("SQ_WAIT", "SQ_ACTIVE_INST")):
                        parts.append(f"{c[3:].lower()}={mean[c] / mean['SQ_WAVE_CYCLES']:.3f}")
            for c in names:
                parts.append(f"{c}={mean[c]:.6g}")
            key = f"{secs[sid][0]}/{label}"
            bound, work = {l: (b, w) for l, b, w in secs[sid][1]}[label]
            for c in ("FETCH_SIZE", "WRITE_SIZE"):
                if c in mean and c in scale:
                    byts = mean[c] * 1024 / scale[c]
                    parts.append(f"{c.split('_')[0].lower()}_MB={byts / 1e6:.1f}")
                    traffic.setdefault(key, {})[c.lower().replace("_size", "_bytes")] = int(byts)
                    if bound == "hbm":
                        traffic[key]["algorithmic_bytes"] = work
            out.append("  ".join(parts))
        out.append("")
    if traffic_json:
        merged = {}
        if os.path.exists(traffic_json):
            with open(traffic_json) as f:
                merged = json.load(f)
        for key, e in traffic.items():
            merged.setdefault(key, {}).update(e)
        for e in merged.values():
            if "fetch_bytes" in e and "write_bytes" in e:
                e["total_bytes"] = e["fetch_bytes"] + e["write_bytes"]
                if "algorithmic_bytes" in e:
                    e["ratio"] = round(e["total_bytes"] / e["algorithmic_bytes"], 3)
        with open(traffic_json, "w") as f:
            json.dump(merged, f, indent=1, sort_keys=True)
    print("\n".join(out))


# ---------------------------------------------------------------------------
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--configs", default="1,2,3,4,5,6,7")
    ap.add_argument("--mark-sections", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 1 GiB streaming copy (calibrates HBM traffic counters)")
    ap.add_argument("--summarize", metavar="DIR", help="summarize rocprofv3 CSV output of a marked run")
    ap.add_argument("--traffic-json", metavar="PATH", help="with --summarize: merge HBM traffic into PATH")
    a = ap.parse_args()
    if a.summarize:
        summarize(a.summarize, a.traffic_json)
        return
    if a.gpus != 1:
        print(f"bench.py runs on exactly one GPU; --gpus {a.gpus} is not supported "
              "(the kernels run on one GPU's share of the work; no multi-GPU leg is implemented)", file=sys.stderr)
        sys.exit(2)
    want = {int(c) for c in a.configs.split(",") if c}
    if 2 not in want:
        want.add(2)  # the headline

    from nkipy_amd.runtime.hip import get_runtime

    rt = get_runtime()
    info = rt.device_info()
    log(f"device {info['arch']} CUs={info['cu_count']} sclk={info['clock_khz'] / 1e6:.2f} GHz")
    mk = Marker(rt, a.mark_sections)
    if a.calibrate_copy:
        calibrate_copy(rt, mk)

    benches = {1: bench_softmax, 2: bench_rmsnorm, 3: bench_swiglu, 4: bench_linattn, 5: bench_decoder,
               6: bench_qwen3_prefill, 7: bench_qwen3_decode}
    entries, legs = {}, {}
    for cid in sorted(want):
        e, leg = benches[cid](a, rt, mk)
        entries[cid], legs[cid] = e, leg
        r = e["roofline"]
        log(f"config {cid} {e['workload']}: {e['us_per_step']} us/step, {r['achieved']} {r['unit']} "
            f"({r['frac'] * 100:.1f}% of {r['peak']:.0f})")
        for k in e["kernels"]:
            log(f"   {k['label']:<20} {k['kernel']:<34} {k['us']:>9.2f} us  {k['achieved']:>8.1f} {k['unit']} "
                f"({k['frac'] * 100:.1f}%)")
    if not a.no_cpu:
        for cid in sorted(want):
            cpu, par = legs[cid]()
            entries[cid]["cpu_baseline"], entries[cid]["parity"] = cpu, par
            log(f"config {cid} cpu baseline: {cpu['value']} {cpu['unit']} ({cpu['sample']}); parity "
                f"max_abs {par['max_abs']:.3e} worst/bar {par['worst_of_bar']} ok={par['ok']}")
    else:
        for cid in sorted(want):
            entries[cid]["cpu_baseline"], entries[cid]["parity"] = None, None

    head = entries[2]
    hr = head["roofline"]
    line = {
        "metric": METRIC,
        "value": round(hr["work_per_launch"] / (head["ms_per_step"] * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded normal / uniform inputs of the workloads' shapes; random-init fp8 weights)",
        "config": {
            "workload": "residual_rmsnorm: x, r bf16 (8192, 4096), w bf16 (4096,), eps 1e-6, fp32 accumulation",
            "rows": RMS_ROWS, "hidden": RMS_N, "parallelism": "single-gpu",
        },
        "roofline": hr,
        "cpu_baseline": head["cpu_baseline"],
        "parity_ok": head["parity"]["ok"] if head["parity"] else None,
        "decoder_layer_fp8_us": entries[5]["value"] if 5 in entries else None,
        "qwen3_prefill_attention_us": entries[6]["us_per_step"] if 6 in entries else None,
        "qwen3_decode_step_us": entries[7]["us_per_step"] if 7 in entries else None,
        "configs": [entries[c] for c in sorted(entries)],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
