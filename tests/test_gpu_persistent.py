"""Persistent device-resident execution: a Qwen3-style attention layer run
the way the reference's Qwen3 model drives it (examples/models/qwen3/
qwen3.py:281-338) -- DeviceTensor inputs and outputs, the KV caches passed
as ``cache_k.must_alias_input`` / ``cache_v.must_alias_input`` and updated
in place across repeated calls, the hidden state written over the layer's
own input buffer, start_pos a device tensor -- checked against the same
kernel run as NumPy on the CPU (the reference's CPU path), and the compiled
artefact reloaded from disk by graph hash in place of a new lowering."""

import numpy as np
import pytest

from nkipy_amd.runtime import BaremetalExecutor, CompiledKernel, DeviceKernel, DeviceTensor

pytestmark = pytest.mark.gpu

B, S, MAXS, HID, H, D, HKV, EPS = 2, 16, 64, 256, 4, 64, 2, 1e-6


def prefill(x, qkv_weight, q_norm_weight, k_norm_weight, cache_k, cache_v, o_weight):
    from nkipy_amd.kernels.qwen3 import qwen3_attention_kernel

    return qwen3_attention_kernel(x, qkv_weight, q_norm_weight, k_norm_weight, EPS, H, D, HKV,
                                  cache_k, cache_v, None, o_weight)


def decode(x, qkv_weight, q_norm_weight, k_norm_weight, cache_k, cache_v, start_pos, o_weight):
    from nkipy_amd.kernels.qwen3 import qwen3_attention_kernel

    return qwen3_attention_kernel(x, qkv_weight, q_norm_weight, k_norm_weight, EPS, H, D, HKV,
                                  cache_k, cache_v, start_pos, o_weight)


def _weights(rng):
    return {"qkv_weight": (rng.standard_normal((HID, (H + 2 * HKV) * D)) * 0.06).astype(np.float32),
            "q_norm_weight": rng.uniform(0.5, 1.5, D).astype(np.float32),
            "k_norm_weight": rng.uniform(0.5, 1.5, D).astype(np.float32),
            "o_weight": (rng.standard_normal((H * D, HID)) * 0.06).astype(np.float32)}


def _layer_inputs(w, x, ck, cv, pos=None):
    ins = {"x": x, **w, "cache_k.must_alias_input": ck, "cache_v.must_alias_input": cv}
    if pos is not None:
        ins["start_pos"] = pos
    return ins


def test_decode_loop_with_aliased_caches(gpu, tmp_path):
    rng = np.random.default_rng(3)
    w = _weights(rng)
    x0 = rng.standard_normal((B, S, HID)).astype(np.float32)
    toks = [rng.standard_normal((B, 1, HID)).astype(np.float32) for _ in range(4)]
    pos0 = np.array([S], np.int32)

    # reference CPU path: the same kernels run as NumPy
    ck_ref = np.zeros((B, MAXS, HKV, D), np.float32)
    cv_ref = np.zeros_like(ck_ref)
    ref_out = [prefill(x0, w["qkv_weight"], w["q_norm_weight"], w["k_norm_weight"], ck_ref, cv_ref, w["o_weight"])]
    for i, t in enumerate(toks):
        ref_out.append(decode(t, w["qkv_weight"], w["q_norm_weight"], w["k_norm_weight"], ck_ref, cv_ref,
                              np.array([S + i], np.int32), w["o_weight"]))

    build = str(tmp_path / "build")
    zeros = np.zeros((B, MAXS, HKV, D), np.float32)
    kp = DeviceKernel.compile_and_load(prefill, x0, w["qkv_weight"], w["q_norm_weight"], w["k_norm_weight"],
                                       zeros, zeros, w["o_weight"], build_dir=build)
    kd = DeviceKernel.compile_and_load(decode, toks[0], w["qkv_weight"], w["q_norm_weight"], w["k_norm_weight"],
                                       zeros, zeros, pos0, w["o_weight"], build_dir=build)
    dw = {k: DeviceTensor.from_numpy(v, name=k) for k, v in w.items()}
    ck = DeviceTensor.from_numpy(zeros, name="cache_k")
    cv = DeviceTensor.from_numpy(zeros, name="cache_v")
    hs = DeviceTensor.from_numpy(x0, name="hidden_states")
    # prefill: the layer output goes over its own input buffer
    kp(inputs=_layer_inputs(dw, hs, ck, cv), outputs={"output0": hs, "cache_k": ck, "cache_v": cv})
    got = [hs.numpy()]
    tok = DeviceTensor.from_numpy(toks[0], name="x")
    pos = DeviceTensor.from_numpy(pos0, name="start_pos")
    for i, t in enumerate(toks):
        tok.write_from_numpy(t)
        pos.write_from_numpy(np.array([S + i], np.int32))
        kd(inputs=_layer_inputs(dw, tok, ck, cv, pos), outputs={"output0": tok, "cache_k": ck, "cache_v": cv})
        got.append(tok.numpy())
    for g, r in zip(got, ref_out):
        np.testing.assert_allclose(g, r, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(ck.numpy(), ck_ref, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(cv.numpy(), cv_ref, rtol=1e-4, atol=1e-5)
    # positions past the last decode step were never written
    assert not ck.numpy()[:, S + len(toks):].any()

    # a new process would find the artefact: drop the in-memory cache and
    # load again -- no lowering happens
    from nkipy_amd.dispatch.artifact import RelocatablePlan
    from nkipy_amd.runtime import device_kernel as dkm

    dkm._LOADED_KERNELS.clear()
    real_lower = DeviceKernel._lower
    DeviceKernel._lower = staticmethod(lambda g: (_ for _ in ()).throw(AssertionError("lowered again")))
    try:
        kd2 = DeviceKernel.compile_and_load(decode, toks[0], w["qkv_weight"], w["q_norm_weight"],
                                            w["k_norm_weight"], zeros, zeros, pos0, w["o_weight"], build_dir=build)
    finally:
        DeviceKernel._lower = real_lower
    assert isinstance(kd2.plan, RelocatablePlan) and kd2 is not kd
    # replay the last decode step on copies of the caches from before it
    ck2 = DeviceTensor.from_numpy(ck.numpy(), name="cache_k")
    cv2 = DeviceTensor.from_numpy(cv.numpy(), name="cache_v")
    last = len(toks) - 1
    tok.write_from_numpy(toks[last])
    pos.write_from_numpy(np.array([S + last], np.int32))
    out2 = kd2(inputs=_layer_inputs(dw, tok, ck2, cv2, pos))
    np.testing.assert_allclose(out2["output0"].numpy(), ref_out[-1], rtol=1e-4, atol=1e-5)
    np.testing.assert_array_equal(out2["cache_k"].numpy(), ck.numpy())


def test_baremetal_executor_runs_compiled_artifact(gpu, tmp_path):
    from nkipy_amd.core import compile as C
    from nkipy_amd.core.trace import NKIPyKernel

    def kern(cache, upd, scale):
        cache[1:3] = upd
        return cache * scale, np.sum(upd, axis=-1)

    cache = np.arange(32, dtype=np.float32).reshape(4, 8)
    upd = -np.ones((2, 8), np.float32)
    scale = np.full((4, 8), 0.5, np.float32)
    tk = NKIPyKernel.trace(kern)
    tk.specialize(cache, upd, scale)
    path = C.compile_to_neff(tk, str(tmp_path), neff_name="kern.neff")
    ck = CompiledKernel(tk, path)
    exp_cache = cache.copy()
    exp = kern(exp_cache, upd, scale)
    with BaremetalExecutor() as ex:
        out = ex.run(ck, cache, upd, scale)
        assert len(out) == 2
        np.testing.assert_array_equal(out[0], exp[0])
        np.testing.assert_array_equal(out[1], exp[1])
        np.testing.assert_array_equal(cache, exp_cache)  # alias written back
        res = ex.benchmark(ck, cache, upd, scale, warmup_iterations=1, benchmark_iterations=3)
        assert res.iterations == 3 and res.mean_ms > 0
    with pytest.raises(FileNotFoundError):
        CompiledKernel(tk, str(tmp_path / "missing.neff"))


def test_bf16_decode_loop_fused_generic_and_reloaded(gpu, tmp_path):
    """The bf16 form: prefill on the fused Qwen3 prefill attention, three
    decode steps on the fused decode-attention kernel with the caches
    aliased in place, against the same graphs lowered onto the generic
    kernels (which follow every traced cast point op by op); then the decode
    artefact reloaded by graph hash (no lowering: relocated argument blocks,
    the runtime position read through a relocated address) replays the last
    step bit for bit."""
    import os

    from parity import assert_close

    from nkipy_amd.core import dtypes as dt
    from nkipy_amd.core.trace import NKIPyKernel
    from nkipy_amd.dispatch.artifact import RelocatablePlan
    from nkipy_amd.dispatch.lower import lower
    from nkipy_amd.dispatch.patterns import default_patterns
    from nkipy_amd.dispatch.patterns_attention import AttentionPattern, DecodeAttentionPattern
    from nkipy_amd.kernels.qwen3 import qwen3_attention_kernel
    from nkipy_amd.runtime import device_kernel as dkm
    from oracle import numerics as N

    Bb, Sb, MAXSb, Hb, Db, HKVb = 2, 128, 256, 4, 128, 2
    HIDb = Hb * Db

    def pre(x, qkv_weight, q_norm_weight, k_norm_weight, cache_k, cache_v, o_weight):
        return qwen3_attention_kernel(x, qkv_weight, q_norm_weight, k_norm_weight, EPS, Hb, Db, HKVb,
                                      cache_k, cache_v, None, o_weight)

    def dec(x, qkv_weight, q_norm_weight, k_norm_weight, cache_k, cache_v, start_pos, o_weight):
        return qwen3_attention_kernel(x, qkv_weight, q_norm_weight, k_norm_weight, EPS, Hb, Db, HKVb,
                                      cache_k, cache_v, start_pos, o_weight)

    rng = np.random.default_rng(17)
    bf = lambda a: dt.to_bf16(N.bf16_round(a))
    w = {"qkv_weight": bf(rng.standard_normal((HIDb, (Hb + 2 * HKVb) * Db)) * 0.05),
         "q_norm_weight": bf(rng.uniform(0.5, 1.5, Db)), "k_norm_weight": bf(rng.uniform(0.5, 1.5, Db)),
         "o_weight": bf(rng.standard_normal((Hb * Db, HIDb)) * 0.05)}
    x0 = bf(rng.standard_normal((Bb, Sb, HIDb)))
    toks = [bf(rng.standard_normal((Bb, 1, HIDb))) for _ in range(3)]
    zeros = bf(np.zeros((Bb, MAXSb, HKVb, Db)))
    pos0 = np.array([Sb], np.int32)
    gp = NKIPyKernel.trace(pre).specialize(x0, w["qkv_weight"], w["q_norm_weight"], w["k_norm_weight"],
                                           zeros, zeros, w["o_weight"])
    gd = NKIPyKernel.trace(dec).specialize(toks[0], w["qkv_weight"], w["q_norm_weight"], w["k_norm_weight"],
                                           zeros, zeros, pos0, w["o_weight"])
    generic = [p for p in default_patterns() if not isinstance(p, (AttentionPattern, DecodeAttentionPattern))]
    build = str(tmp_path / "build")
    kinds = {}
    results = {}
    for mode in ("fused", "generic"):
        if mode == "fused":
            kp = DeviceKernel.compile_and_load(pre, x0, w["qkv_weight"], w["q_norm_weight"], w["k_norm_weight"],
                                               zeros, zeros, w["o_weight"], build_dir=build)
            kd = DeviceKernel.compile_and_load(dec, toks[0], w["qkv_weight"], w["q_norm_weight"],
                                               w["k_norm_weight"], zeros, zeros, pos0, w["o_weight"],
                                               build_dir=build)
        else:
            kp = DeviceKernel(gp, lower(gp, generic), "pre_generic")
            kd = DeviceKernel(gd, lower(gd, generic), "dec_generic")
        kinds[mode] = (kp.plan.kernel_kinds, kd.plan.kernel_kinds)
        dw = {k: DeviceTensor.from_numpy(v, name=k) for k, v in w.items()}
        ck = DeviceTensor.from_numpy(zeros, name="cache_k")
        cv = DeviceTensor.from_numpy(zeros, name="cache_v")
        hs = DeviceTensor.from_numpy(x0, name="hidden_states")
        kp(inputs=_layer_inputs(dw, hs, ck, cv), outputs={"output0": hs, "cache_k": ck, "cache_v": cv})
        outs = [hs.numpy()]
        tok = DeviceTensor.from_numpy(toks[0], name="x")
        pos = DeviceTensor.from_numpy(pos0, name="start_pos")
        for i, t in enumerate(toks):
            if i == len(toks) - 1:
                before = (ck.numpy(), cv.numpy())
            tok.write_from_numpy(t)
            pos.write_from_numpy(np.array([Sb + i], np.int32))
            kd(inputs=_layer_inputs(dw, tok, ck, cv, pos), outputs={"output0": tok, "cache_k": ck, "cache_v": cv})
            outs.append(tok.numpy())
        results[mode] = (outs, ck.numpy(), cv.numpy(), before, dw, kd)
    assert "attention" in kinds["fused"][0] and "dot" not in kinds["fused"][0], kinds
    assert "decode_attention" in kinds["fused"][1], kinds
    assert "attention" not in kinds["generic"][0] and "decode_attention" not in kinds["generic"][1]
    name = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    f_outs, f_ck, f_cv, before, dw, kd = results["fused"]
    g_outs, g_ck, g_cv = results["generic"][:3]
    for i, (a, b) in enumerate(zip(f_outs, g_outs)):
        assert_close(dt.to_float32(a), dt.to_float32(b), f"{name} [step {i}]", axis=-1)
    # prefill writes the caches from the same projection / norm / rotary
    # kernels in both lowerings; later rows come from the decode steps
    np.testing.assert_array_equal(dt.numpy_storage(f_ck)[:, :Sb], dt.numpy_storage(g_ck)[:, :Sb])
    assert not dt.numpy_storage(f_ck)[:, Sb + len(toks):].any()

    dkm._LOADED_KERNELS.clear()
    real_lower = DeviceKernel._lower
    DeviceKernel._lower = staticmethod(lambda g: (_ for _ in ()).throw(AssertionError("lowered again")))
    try:
        kd2 = DeviceKernel.compile_and_load(dec, toks[0], w["qkv_weight"], w["q_norm_weight"], w["k_norm_weight"],
                                            zeros, zeros, pos0, w["o_weight"], build_dir=build)
    finally:
        DeviceKernel._lower = real_lower
    assert isinstance(kd2.plan, RelocatablePlan) and kd2 is not kd
    assert "decode_attention" in kd2.plan.kernel_kinds and repr(kd2).startswith("DeviceKernel(")
    ck2 = DeviceTensor.from_numpy(before[0], name="cache_k")
    cv2 = DeviceTensor.from_numpy(before[1], name="cache_v")
    tok = DeviceTensor.from_numpy(toks[-1], name="x")
    pos = DeviceTensor.from_numpy(np.array([Sb + len(toks) - 1], np.int32), name="start_pos")
    out2 = kd2(inputs=_layer_inputs(dw, tok, ck2, cv2, pos))
    np.testing.assert_array_equal(dt.numpy_storage(out2["output0"].numpy()), dt.numpy_storage(f_outs[-1]))
    np.testing.assert_array_equal(dt.numpy_storage(out2["cache_k"].numpy()), dt.numpy_storage(f_ck))
    np.testing.assert_array_equal(dt.numpy_storage(out2["cache_v"].numpy()), dt.numpy_storage(f_cv))


def test_bf16_decode_loop_graph_replay_equals_launches(gpu, tmp_path):
    """The fused bf16 decode step replayed as one HIP graph (captured on the
    first call with the loop's tensors, reused on every later step, the
    token and position rewritten in place between steps) equals the same
    step launched one kernel at a time on a second copy of the caches, bit
    for bit at every step, with the eager step and a synchronisation between
    consecutive replays."""
    import ctypes

    from nkipy_amd.core import dtypes as dt
    from nkipy_amd.kernels.qwen3 import qwen3_attention_kernel
    from nkipy_amd.runtime.hip import SpikeError, _check, get_runtime
    from oracle import numerics as N

    Bb, Sb, MAXSb, Hb, Db, HKVb = 2, 64, 256, 4, 128, 2
    HIDb = Hb * Db

    def pre(x, qkv_weight, q_norm_weight, k_norm_weight, cache_k, cache_v, o_weight):
        return qwen3_attention_kernel(x, qkv_weight, q_norm_weight, k_norm_weight, EPS, Hb, Db, HKVb,
                                      cache_k, cache_v, None, o_weight)

    def dec(x, qkv_weight, q_norm_weight, k_norm_weight, cache_k, cache_v, start_pos, o_weight):
        return qwen3_attention_kernel(x, qkv_weight, q_norm_weight, k_norm_weight, EPS, Hb, Db, HKVb,
                                      cache_k, cache_v, start_pos, o_weight)

    rng = np.random.default_rng(29)
    bf = lambda a: dt.to_bf16(N.bf16_round(a))
    w = {"qkv_weight": bf(rng.standard_normal((HIDb, (Hb + 2 * HKVb) * Db)) * 0.05),
         "q_norm_weight": bf(rng.uniform(0.5, 1.5, Db)), "k_norm_weight": bf(rng.uniform(0.5, 1.5, Db)),
         "o_weight": bf(rng.standard_normal((Hb * Db, HIDb)) * 0.05)}
    x0 = bf(rng.standard_normal((Bb, Sb, HIDb)))
    toks = [bf(rng.standard_normal((Bb, 1, HIDb))) for _ in range(5)]
    zeros = bf(np.zeros((Bb, MAXSb, HKVb, Db)))
    pos0 = np.array([Sb], np.int32)
    build = str(tmp_path / "build")
    kp = DeviceKernel.compile_and_load(pre, x0, w["qkv_weight"], w["q_norm_weight"], w["k_norm_weight"],
                                       zeros, zeros, w["o_weight"], build_dir=build)
    kd = DeviceKernel.compile_and_load(dec, toks[0], w["qkv_weight"], w["q_norm_weight"], w["k_norm_weight"],
                                       zeros, zeros, pos0, w["o_weight"], build_dir=build)
    assert "decode_attention" in kd.plan.kernel_kinds, kd.plan.kernel_kinds
    dw = {k: DeviceTensor.from_numpy(v, name=k) for k, v in w.items()}
    sets = []
    for _ in range(2):
        ck = DeviceTensor.from_numpy(zeros, name="cache_k")
        cv = DeviceTensor.from_numpy(zeros, name="cache_v")
        hs = DeviceTensor.from_numpy(x0, name="hidden_states")
        kp(inputs=_layer_inputs(dw, hs, ck, cv), outputs={"output0": hs, "cache_k": ck, "cache_v": cv})
        sets.append((ck, cv, DeviceTensor.from_numpy(toks[0], name="x"),
                     DeviceTensor.from_numpy(pos0, name="start_pos")))
    graphs = set()
    for i, t in enumerate(toks):
        outs = []
        for (ck, cv, tok, pos), graph in zip(sets, (False, True)):
            tok.write_from_numpy(t)
            pos.write_from_numpy(np.array([Sb + i], np.int32))
            kd(inputs=_layer_inputs(dw, tok, ck, cv, pos), outputs={"output0": tok, "cache_k": ck, "cache_v": cv},
               graph=graph)
            outs.append((tok.numpy(), ck.numpy(), cv.numpy()))
        graphs |= {bp._graph for bp in kd.executor._bound.values() if bp._graph is not None}
        for what, a, b in zip(("output", "cache_k", "cache_v"), *outs):
            np.testing.assert_array_equal(dt.numpy_storage(b), dt.numpy_storage(a), err_msg=f"step {i} {what}")
    assert len(graphs) == 1, graphs  # captured once, replayed on every later step
    rt = get_runtime()
    with pytest.raises(SpikeError, match="not a live graph"):
        _check(rt.lib.nkh_graph_launch(ctypes.c_void_p(16)), "graph launch")
    bound = list(kd.executor._bound.values())
    kd.executor.close()  # releases the captured graph
    assert bound and all(bp._graph is None for bp in bound)
    with pytest.raises(SpikeError, match="not a live graph"):
        _check(rt.lib.nkh_graph_destroy(ctypes.c_void_p(graphs.pop())), "graph release")
