"""Host-side tests (no GPU): the C-ABI library and its exports, the tracer's
naming and promotion contract, strided views, pattern lowering of every
hot-path kernel at its workload shape, and the launchers' operand checks."""

import ctypes
import os
import re

import numpy as np
import pytest

from nkipy_amd import _build
from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.backend import promotion as P
from nkipy_amd.core.trace import NKIPyKernel
from nkipy_amd.dispatch import launchers as LA
from nkipy_amd.dispatch.lower import lower
from nkipy_amd.dispatch.views import resolve

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


# ---------------------------------------------------------------------------
# C ABI
# ---------------------------------------------------------------------------
def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "nkipy_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nkh_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    path = _build.RUNTIME_LIB
    assert path.exists(), "build the runtime first (__graft_entry__.build())"
    lib = ctypes.CDLL(str(path))
    names = _declared_symbols()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_last_error_and_uninitialised_calls_fail_cleanly():
    lib = ctypes.CDLL(str(_build.RUNTIME_LIB))
    lib.nkh_last_error.restype = ctypes.c_char_p
    flag = ctypes.c_int(-1)
    assert lib.nkh_is_initialized(ctypes.byref(flag)) == 0
    if flag.value == 0:
        # device calls before nkh_init report NOT_INIT instead of touching HIP
        assert lib.nkh_sync() == 3
        assert b"init" in lib.nkh_last_error().lower()


def test_no_kernel_uses_scratch_memory():
    """Register spills or private arrays left in memory would put scratch
    traffic into the kernels' inner loops."""
    import json

    # SwiGLU epilogues that hold both products at once (spill outside the
    # K loop); the 4-wave kernels are not the default path
    known = {"nk_gemm8_swiglu_nt_e4m3_bf16", "nk_gemm_swiglu_nn_bf16_bf16", "nk_gemm_swiglu_nt_e4m3_bf16"}
    for src in _build.kernel_sources():
        man = json.loads(_build.hsaco_path(src.stem).with_suffix(".json").read_text())
        for name, meta in man.items():
            if name in known:
                continue
            assert meta.get("scratch", 0) == 0 and meta.get("vgpr_spill", 0) == 0, (name, meta)


def test_every_kernel_object_has_a_manifest():
    for src in _build.kernel_sources():
        hsaco = _build.hsaco_path(src.stem)
        assert hsaco.exists(), hsaco
        assert hsaco.with_suffix(".json").exists()


# ---------------------------------------------------------------------------
# promotion rules (expectations of tests/unit/test_type_promotion.py)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("t0,t1,expected", [
    (dt.bool_, dt.int32, dt.int32), (dt.bool_, dt.float32, dt.float32),
    (dt.bool_, P.WEAK_INT, dt.int32), (dt.bool_, P.WEAK_FLOAT, dt.float32),
    (P.WEAK_INT, dt.int8, dt.int8), (P.WEAK_INT, dt.float32, dt.float32),
    (P.WEAK_FLOAT, dt.int32, dt.float32), (P.WEAK_FLOAT, dt.float16, dt.float16),
    (dt.int8, dt.int16, dt.int16), (dt.int32, dt.int64, dt.int64), (dt.uint8, dt.uint32, dt.uint32),
    (dt.int8, dt.uint8, dt.int16), (dt.int32, dt.uint64, dt.float32),
    (dt.float16, dt.float32, dt.float32), (dt.float16, dt.bfloat16, dt.float32),
    (P.WEAK_FLOAT, dt.bfloat16, dt.bfloat16), (dt.bfloat16, dt.float32, dt.float32),
])
def test_promotion_table_samples(t0, t1, expected):
    assert P.lookup(t0, t1) == expected
    assert P.lookup(t1, t0) == expected


def test_promotion_keys_and_common_types():
    assert P.type_key(True) == dt.bool_
    assert P.type_key(3) is P.WEAK_INT and P.type_key(2.5) is P.WEAK_FLOAT
    assert P.type_key(np.int32(5)) == dt.int32
    assert P.find_common_type(np.array([True, False]), 1000) == dt.int32
    assert P.find_common_type(np.array([1, 2], np.int8), 100) == dt.int8
    assert P.find_common_type(np.array([1, 2], np.int8), 3.14) == dt.float32
    with pytest.raises(TypeError):
        P.lookup(dt.float32, np.dtype(np.float64))  # float64 is rejected, not narrowed
    assert P.lookup(dt.float8_e4m3fn, dt.int32) == dt.float8_e4m3fn


# ---------------------------------------------------------------------------
# tracer naming contract
# ---------------------------------------------------------------------------
def test_trace_names_inputs_outputs_and_aliases():
    def kern(a, b):
        a[0] = b[0]          # mutates a: a.must_alias_input, result named "a"
        return a * 2, b + 1  # other results: output{i}

    x = np.zeros((4, 8), np.float32)
    g = NKIPyKernel.trace(kern).specialize(x, x.copy())
    pnames = [p.name for p in g.parameters]
    assert pnames == ["a.must_alias_input", "b"]
    rnames = [r.name for r in g.results]
    assert "a" in rnames and "output0" in rnames and "output1" in rnames


# ---------------------------------------------------------------------------
# strided views
# ---------------------------------------------------------------------------
def test_view_of_split_repeat_transpose():
    B, S = 2, 5

    def f(qkv):
        q, k, v = np.split(qkv, [64, 80], axis=-1)
        vv = np.repeat(v.reshape(B, S, 2, 8), 4, axis=2).transpose(0, 2, 1, 3)
        kk = np.repeat(k.reshape(B, S, 2, 8), 4, axis=2).transpose(0, 2, 3, 1)
        return vv * 1.0, kk * 1.0

    x = np.arange(B * S * 96, dtype=np.float32).reshape(B, S, 96)
    g = NKIPyKernel.trace(f).specialize(x)
    q, k, v = np.split(x, [64, 80], axis=-1)
    refs = (np.repeat(v.reshape(B, S, 2, 8), 4, axis=2).transpose(0, 2, 1, 3),
            np.repeat(k.reshape(B, S, 2, 8), 4, axis=2).transpose(0, 2, 3, 1))
    for r, ref in zip(g.results, refs):
        op = r.node.inputs[0] if r.node.inputs[0].ndim == 4 else r.node.inputs[1]
        vw = resolve(op)
        assert vw.base.shape == x.shape
        np.testing.assert_array_equal(vw.materialize_check(x), ref)
        assert vw.grouped(1) == (2, 8, 4)  # 2 KV heads, stride 8, each repeated 4x


def test_view_reshape_merge_and_split():
    def f(x):
        return x.reshape(12, 10) * 2.0, x[:, 1:5, :].reshape(2, 4, 2, 5) * 2.0

    x = np.arange(120, dtype=np.float32).reshape(2, 6, 10)
    g = NKIPyKernel.trace(f).specialize(x)
    refs = (x.reshape(12, 10), x[:, 1:5, :].reshape(2, 4, 2, 5))
    for r, ref in zip(g.results, refs):
        op = next(v for v in r.node.inputs if v.shape == ref.shape and v.size > 1)
        vw = resolve(op)
        assert vw.base.is_parameter
        np.testing.assert_array_equal(vw.materialize_check(x), ref)


# ---------------------------------------------------------------------------
# pattern lowering at the workload shapes
# ---------------------------------------------------------------------------
def _bf16(shape):
    return np.zeros(shape, dt.bfloat16)


def _fp8(shape):
    return np.zeros(shape, np.uint8).view(dt.float8_e4m3fn)


def _kinds(fn, *args, **kw):
    plan = lower(NKIPyKernel.trace(fn).specialize(*args, **kw))
    _assert_temps_written_before_read(plan)
    return plan.kernel_kinds


def test_lowering_softmax_and_rmsnorm():
    from nkipy_amd.kernels import residual_rmsnorm_kernel, rmsnorm_kernel, softmax_kernel

    assert _kinds(softmax_kernel, np.zeros((2048, 4096), np.float32)) == ["softmax"]
    assert _kinds(residual_rmsnorm_kernel, _bf16((8192, 4096)), _bf16((8192, 4096)), _bf16((4096,)),
                  1e-6) == ["rmsnorm"]
    assert _kinds(rmsnorm_kernel, _bf16((64, 4096)), _bf16((4096,)), 1e-6) == ["rmsnorm"]


def test_lowering_swiglu_and_linear_attention():
    from nkipy_amd.kernels import chunked_linear_attention_kernel, feedforward_kernel, swiglu_mlp_kernel

    assert _kinds(swiglu_mlp_kernel, _bf16((4096, 4096)), _bf16((4096, 14336)), _bf16((4096, 14336)),
                  _bf16((14336, 4096))) == ["gemm_swiglu", "gemm"]
    assert _kinds(feedforward_kernel, _bf16((256, 512)), _bf16((512, 2048)), _bf16((1024, 512))) == \
        ["gemm_swiglu", "gemm"]
    q = _bf16((4, 16, 8192, 128))
    assert _kinds(chunked_linear_attention_kernel, q, q, q) == ["linear_attention"]
    # fp32 inputs are not the kernel's dtype: generic lowering, no fused step
    f = np.zeros((1, 2, 128, 16), np.float32)
    kinds = _kinds(chunked_linear_attention_kernel, f, f, f, 32)
    assert "linear_attention" not in kinds and kinds


def test_lowering_decoder_layer_fp8():
    from nkipy_amd.kernels import llama_decoder_layer_fp8

    B, S, Hq, Hkv, D, F = 8, 2048, 32, 8, 128, 14336
    hid = Hq * D
    one = lambda n: np.ones(n, np.float32)
    args = [_bf16((B, S, hid)), _bf16((hid,)), _fp8(((Hq + 2 * Hkv) * D, hid)), one((Hq + 2 * Hkv) * D),
            _fp8((hid, hid)), one(hid), _bf16((hid,)), _fp8((F, hid)), one(F), _fp8((F, hid)), one(F),
            _fp8((hid, F)), one(hid)]
    assert _kinds(llama_decoder_layer_fp8, *args) == [
        "rmsnorm", "gemm_rope", "attention", "gemm", "rmsnorm", "gemm_swiglu", "gemm"]


def _assert_temps_written_before_read(plan):
    """Every temporary a step reads is written by an earlier step."""
    written = set()
    for st in plan.steps:
        for v in st.inputs:
            b = plan.slot(v).buffer
            if plan.buffers[b].kind == "temp":
                assert b in written, f"step {st.desc} reads temporary {b} ({v!r}) before any step writes it"
        written.update(plan.slot(v).buffer for v in st.outputs)


def test_lowering_value_inside_a_match_read_through_a_view():
    """``(h @ w).astype(bf16)`` with bf16 operands: the GEMM absorbs the
    no-op cast, and the RoPE views look through it to the product itself,
    which must then share the GEMM output's storage."""
    from nkipy_amd.dispatch.patterns import default_patterns
    from nkipy_amd.dispatch.patterns_attention import QkvRopeFusion
    from nkipy_amd.kernels.decoder import rope_kernel, rope_tables

    B, S, H, D, hid = 1, 64, 2, 128, 128
    cos, sin = rope_tables(D, S, 1e4)

    def fn(h, w):
        q = np.matmul(h, w).astype(h.dtype)
        return rope_kernel(q.reshape(B, S, H, D), cos, sin).astype(h.dtype)

    g = NKIPyKernel.trace(fn).specialize(_bf16((B, S, hid)), _bf16((hid, H * D)))
    plain = lower(g, [p for p in default_patterns() if not isinstance(p, QkvRopeFusion)])
    assert plain.kernel_kinds == ["gemm", "rope"]
    _assert_temps_written_before_read(plain)


def test_lowering_qkv_rope_fusion_only_when_qk_columns_are_private():
    """RoPE folds into the QKV projection only when nothing else reads the
    q / k columns the fused epilogue leaves unwritten."""
    from nkipy_amd.kernels.decoder import rope_kernel, rope_tables

    B, S, Hq, Hkv, D, hid = 2, 128, 4, 2, 128, 256
    cos, sin = rope_tables(D, S, 1e4)
    x, w = _bf16((B, S, hid)), _bf16((hid, (Hq + 2 * Hkv) * D))

    def qkv_rope(extra):
        def fn(h, w):
            qkv = np.matmul(h, w).astype(h.dtype)
            q, k, v = np.split(qkv, [Hq * D, (Hq + Hkv) * D], axis=-1)
            qr = rope_kernel(q.reshape(B, S, Hq, D), cos, sin).astype(h.dtype)
            kr = rope_kernel(k.reshape(B, S, Hkv, D), cos, sin).astype(h.dtype)
            outs = [qr, kr, v.reshape(B, S, Hkv, D)]
            if extra == "raw_k":
                outs.append(k * 2.0)
            elif extra == "qkv":
                outs.append(qkv)
            elif extra == "v_sum":
                outs.append(np.sum(v.astype(np.float32), axis=-1))
            return tuple(outs)
        return fn

    assert _kinds(qkv_rope(None), x, w)[0] == "gemm_rope"
    _assert_temps_written_before_read(lower(NKIPyKernel.trace(qkv_rope(None)).specialize(x, w)))
    assert _kinds(qkv_rope("v_sum"), x, w)[0] == "gemm_rope"   # v columns only
    for extra in ("raw_k", "qkv"):
        kinds = _kinds(qkv_rope(extra), x, w)
        assert "gemm_rope" not in kinds and kinds.count("rope") == 2, (extra, kinds)


def test_lowering_attention_variants_and_non_matches():
    from nkipy_amd.kernels import causal_gqa_attention_kernel
    from nkipy_amd.kernels.softmax import softmax_kernel

    q = _bf16((1, 256, 8, 128))
    assert _kinds(causal_gqa_attention_kernel, q, _bf16((1, 256, 1, 128)), _bf16((1, 256, 1, 128))) == \
        ["attention"]   # one KV head shared by all (stride 0)
    assert _kinds(causal_gqa_attention_kernel, q, q, q) == ["attention"]  # no GQA

    def anti_causal(xq, xk, xv):  # mask on the wrong side: not the causal kernel
        S, D = xq.shape[1], xq.shape[3]
        q = xq.transpose(0, 2, 1, 3).astype(np.float32)
        k = xk.transpose(0, 2, 3, 1).astype(np.float32)
        v = xv.transpose(0, 2, 1, 3).astype(np.float32)
        s = np.matmul(q, k) / np.float32(np.sqrt(D)) + np.tril(np.full((S, S), -1e5, np.float32), k=-1)
        return np.matmul(softmax_kernel(s), v).astype(xq.dtype)

    kinds = _kinds(anti_causal, q, q, q)
    assert "attention" not in kinds and "dot" in kinds

    def head_dim_64(xq, xk, xv):
        return causal_gqa_attention_kernel(xq, xk, xv)

    q64 = _bf16((1, 256, 2, 64))
    assert "attention" not in _kinds(head_dim_64, q64, q64, q64)


# ---------------------------------------------------------------------------
# launcher operand checks (host side, nothing launched)
# ---------------------------------------------------------------------------
def test_launchers_reject_operands_the_kernels_cannot_take():
    A = 1 << 20
    with pytest.raises(LA.LaunchError):
        LA.gemm(A, A, A, 64, 64, 12, layout="nt", b_dtype=dt.bfloat16, c_dtype=dt.bfloat16)  # K % 8
    with pytest.raises(LA.LaunchError):
        LA.gemm(A, A, A, 64, 64, 24, layout="nt", b_dtype=dt.float8_e4m3fn, c_dtype=dt.bfloat16,
                scale_ptr=A)  # fp8 NT needs K % 16
    with pytest.raises(LA.LaunchError):
        LA.gemm(A + 4, A, A, 64, 64, 64, layout="nn", b_dtype=dt.bfloat16, c_dtype=dt.bfloat16)  # align
    st = {n: (256 * 128, 128, 128) for n in "qkvo"}
    with pytest.raises(LA.LaunchError):
        LA.attention(A, A, A, A, 1, 200, 1, 1, 128, 0.1, st)  # S % 128
    with pytest.raises(LA.LaunchError):
        LA.attention(A, A, A, A, 1, 256, 1, 1, 64, 0.1, st)  # head dim
    with pytest.raises(LA.LaunchError):
        LA.linear_attention(A, A, A, A, 4, 100)  # T % 64
    with pytest.raises(LA.LaunchError):
        LA.rope(A, A, A, A, 1, 8, 2, 128, (1024, 256, 130), (1024, 256, 128), 64, 64)  # stride alignment
    ok = LA.gemm(A, A, A, 300, 520, 136, layout="nn", b_dtype=dt.bfloat16, c_dtype=dt.bfloat16)
    assert ok.grid[0] == 2 * 3 and ok.flops == 2 * 300 * 520 * 136


def test_few_row_projection_forms_split_and_route():
    """The MFMA few-row projection: K ranges of 256 while the grid fits one
    round of 512 workgroups, else the shortest multiple of 32 that fits (at
    most 512 for 16 rows, 256 for 32); ranges cover K; routing up to 16
    rows, and 32 while ranges of 256 fit one round; operand checks."""
    A = 1 << 20
    assert LA.gemv_mfma_split(8, 6144, 4096) == (16, 256)
    assert LA.gemv_mfma_split(8, 4096, 14336) == (32, 448)
    assert LA.gemv_mfma_split(8, 24576, 4096) == (8, 512)
    assert LA.gemv_mfma_split(32, 4096, 14336) == (56, 256)
    for M, N, K in ((1, 6144, 4096), (13, 1000, 328), (8, 151936, 4096), (17, 520, 2056), (5, 264, 8)):
        ks, kc = LA.gemv_mfma_split(M, N, K)
        assert kc % 32 == 0 and kc <= (512 if M <= 16 else 256)
        assert (ks - 1) * kc < K <= ks * kc
        launches = LA.gemv_mfma(A, A, A, M, N, K, c_dtype=dt.bfloat16, ws_ptr=A)
        assert [l.symbol for l in launches] == [f"nk_gemv_mfma_nn_bf16_t{1 if M <= 16 else 2}",
                                                "nk_gemv_out_bf16"]
        assert launches[0].grid[0] == -(-N // 256) * ks
        assert LA.gemv_mfma_workspace_bytes(M, N, K) == 4 * ks * M * N
    assert LA.gemv_mfma_split(8, 14336, 4096, swiglu=True) == (8, 512)  # 112 blocks of 128 columns
    assert LA.gemv_mfma_workspace_bytes(8, 1536, 2048, swiglu=True) == 2 * 4 * 8 * 8 * 1536
    sw = LA.gemv_mfma(A, A, A, 8, 1536, 2048, c_dtype=dt.bfloat16, ws_ptr=A, up_ptr=A + 3072, ldb=3072)
    assert [l.symbol for l in sw] == ["nk_gemv_mfma_nn_bf16_swiglu_t1", "nk_gemv_out_bf16_swiglu"]
    assert sw[0].grid[0] == 12 * 8
    with pytest.raises(LA.LaunchError):
        LA.gemv_mfma(A, A, A, 8, 64, 64, c_dtype=dt.bfloat16, ws_ptr=A, up_ptr=A, bias_ptr=A)  # SwiGLU + bias
    assert LA.gemv_mfma_preferred(1, 4096, 4096) and LA.gemv_mfma_preferred(16, 24576, 14336)
    assert LA.gemv_mfma_preferred(32, 6144, 4096) and not LA.gemv_mfma_preferred(32, 4096, 14336)
    assert not LA.gemv_mfma_preferred(33, 64, 64) and not LA.gemv_mfma_preferred(0, 64, 64)
    # NT weights: one row stays on the VALU form; no fp8 NN form
    assert not LA.gemv_mfma_preferred(1, 4096, 4096, layout="nt")
    assert LA.gemv_mfma_preferred(2, 4096, 4096, layout="nt", fp8=True)
    assert not LA.gemv_mfma_preferred(8, 4096, 4096, layout="nn", fp8=True)
    nt = LA.gemv_mfma(A, A, A, 8, 1000, 336, c_dtype=dt.bfloat16, ws_ptr=A, layout="nt",
                      b_dtype=dt.float8_e4m3fn, scale_ptr=A)
    assert [l.symbol for l in nt] == ["nk_gemv_mfma_nt_e4m3_t1", "nk_gemv_out_bf16"] and nt[0].args.flags & LA.GEMM_SCALE
    with pytest.raises(LA.LaunchError):
        LA.gemv_mfma(A, A, A, 8, 1000, 328, c_dtype=dt.bfloat16, ws_ptr=A, layout="nt",
                     b_dtype=dt.float8_e4m3fn, scale_ptr=A)  # fp8 K % 16
    with pytest.raises(LA.LaunchError):
        LA.gemv_mfma(A, A, A, 8, 1000, 336, c_dtype=dt.bfloat16, ws_ptr=A, layout="nt",
                     b_dtype=dt.float8_e4m3fn)  # fp8 without scales
    with pytest.raises(LA.LaunchError):
        LA.gemv_mfma(A, A, A, 8, 1024, 1024, c_dtype=dt.bfloat16, ws_ptr=A, b_dtype=dt.float8_e4m3fn,
                     scale_ptr=A)  # fp8 NN
    with pytest.raises(LA.LaunchError):
        LA.gemv_mfma(A, A, A, 33, 64, 64, c_dtype=dt.bfloat16, ws_ptr=A)  # rows
    with pytest.raises(LA.LaunchError):
        LA.gemv_mfma(A, A, A, 8, 60, 64, c_dtype=dt.bfloat16, ws_ptr=A)  # N % 8
    with pytest.raises(LA.LaunchError):
        LA.gemv_mfma(A, A + 8, A, 8, 64, 64, c_dtype=dt.bfloat16, ws_ptr=A)  # weight alignment
    with pytest.raises(LA.LaunchError):
        LA.gemv_mfma(A, A, A, 8, 64, 64, c_dtype=dt.bfloat16, ws_ptr=0)  # workspace
    with pytest.raises(LA.LaunchError):
        LA.gemv_mfma(A, A, A, 8, 64, 64, c_dtype=dt.float16, ws_ptr=A)  # output dtype


# ---------------------------------------------------------------------------
# in-place aliasing: a deferred read of a mutated parameter must not see the update
# ---------------------------------------------------------------------------
def _alias_plan(fn, *args):
    return lower(NKIPyKernel.trace(fn).specialize(*args))


def test_alias_deferred_reader_forces_staged_write_back():
    def kern(cache, new):
        old = cache * 2.0          # fused into the later add: reads cache late
        cache[0:1] = new
        return old + 1.0

    plan = _alias_plan(kern, np.zeros((4, 8), np.float32), np.ones((1, 8), np.float32))
    descs = [s.desc for s in plan.steps]
    # the update goes to a staging temporary, and the caller's buffer is
    # written back after every step that reads the old contents
    assert descs[-1].startswith("write back"), descs
    staged = [b for b in plan.buffers if b.name.endswith(".staged")]
    assert len(staged) == 1


def test_alias_materialised_earlier_reader_keeps_in_place_update():
    def kern(cache, new):
        s = np.sum(cache, axis=1)  # materialised reduce, runs before the update
        cache[0:1] = new
        return s

    plan = _alias_plan(kern, np.zeros((4, 8), np.float32), np.ones((1, 8), np.float32))
    descs = [s.desc for s in plan.steps]
    assert not any(d.startswith("write back") for d in descs), descs
    assert not any(b.name.endswith(".staged") for b in plan.buffers)


def test_alias_update_reading_its_own_target_is_not_in_place_read():
    def kern(cache):
        cache[1:3] = cache[0:2]  # overlapping read and write of one buffer
        return cache

    plan = _alias_plan(kern, np.zeros((4, 8), np.float32))
    descs = [s.desc for s in plan.steps]
    # the source rows are copied out (or the update staged) before the
    # buffer is written, never read by the updating step itself
    assert descs[-1].startswith("write back") or (len(descs) == 2 and descs[1] == "update slice"), descs


# ---------------------------------------------------------------------------
# C-ABI linear attention: the library's work split equals the launcher's
# ---------------------------------------------------------------------------
def test_c_abi_linear_attention_workspace_matches_launcher():
    from nkipy_amd.runtime.hip import load_library

    lib = load_library()
    size = ctypes.c_size_t()
    for bh in (1, 2, 3, 4, 16, 64, 255, 256, 1024):
        for t in (64, 128, 512, 1024, 4096, 8192, 16384, 65536):
            assert lib.nkh_linear_attention_workspace_size(bh, t, ctypes.byref(size)) == 0
            assert size.value == LA.linear_attention_workspace_bytes(bh, t), (bh, t)
    for bh, t in ((0, 64), (4, 100), (4, 0), (-1, 64)):
        assert lib.nkh_linear_attention_workspace_size(bh, t, ctypes.byref(size)) == 2
        assert b"multiple of 64" in lib.nkh_last_error()


def test_profile_ranges_need_no_device_and_reject_unbalanced_pops():
    from nkipy_amd.runtime.hip import SpikeError, load_library, profile_range

    with profile_range("outer") as have:
        assert have in (True, False)
        with profile_range("inner"):
            pass
    lib = load_library()
    assert lib.nkh_profile_range_pop() != 0
    assert b"without a push" in lib.nkh_last_error()


def test_divide_rounds_as_multiply_is_checked_per_divisor():
    """A score divided by c and rounded to bf16 equals the product by
    RN(1 / c) rounded to bf16 for every bf16 score when c = sqrt(128), not
    when c sits next to a ratio of a bf16 significand and a rounding
    midpoint; the launcher keeps the correctly rounded divide then."""
    rng = np.random.default_rng(0)
    s = dt.round_to_bf16(rng.standard_normal(1 << 16).astype(np.float32) * 30)
    for c, same in ((float(np.sqrt(128)), True), (3.0188679695129395, False)):
        assert LA.divide_rounds_as_multiply(c) is same
        if same:  # spot check of the claim on random scores
            np.testing.assert_array_equal(dt.round_to_bf16(s / np.float32(c)),
                                          dt.round_to_bf16(s * (np.float32(1) / np.float32(c))))
        st = {"q": (8 * 128, 128, 8 * 128), "k": (8 * 128, 128, 0), "v": (8 * 128, 128, 0),
              "o": (8 * 128, 128, 8 * 128)}
        (_, _, l) = LA.attention(1 << 20, 1 << 20, 1 << 20, 1 << 20, 1, 256, 1, 1, 128, 1 / c, st,
                                 score_flags=LA.ATT_RND_PROD | LA.ATT_RND_SCORE | LA.ATT_DIVIDE | LA.ATT_SOFTMAX_BF16,
                                 divisor=c, rowstat_ptr=1 << 20)
        assert bool(l.args.flags & LA.ATT_DIVIDE) is not same
        # the decode step: the same rewrite when the product and the score
        # are rounded; an fp32 product keeps the divide
        dst = {"q": (128, 128), "k": (128, 128, 128), "v": (128, 128, 128), "o": (128, 128)}
        for flags, rewrite in ((LA.DEC_RND_PROD | LA.DEC_RND_SCORE | LA.DEC_SOFTMAX_BF16, same),
                               (LA.DEC_RND_SCORE, False)):
            ls = LA.decode_attention(1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 1, 256, 1, 1, 128, c, dst,
                                     flags=flags | LA.DEC_DIVIDE, ws_ptr=1 << 20)
            a = ls[0].args
            assert bool(a.flags & LA.DEC_DIVIDE) is not rewrite
            assert np.float32(a.scale) == (np.float32(1) / np.float32(c) if rewrite else np.float32(c))


def test_lowering_qwen3_head_prologue_is_one_launch():
    """The Qwen3 attention prologue (split of the QKV projection, per-head
    q / k RMSNorm, tables cast to bf16 and taken at the runtime position,
    bf16-step RoPE, the k / v cache writes at that position) lowers to one
    head_rope launch that reads the projection's partial sums in place and
    the fp32 tables directly and writes k and v into the caches' rows: the
    decode layer is the two projections around it and the attention."""
    from nkipy_amd.kernels.qwen3 import qwen3_attention_kernel

    B, MAXS, HID, H, D, HKV = 2, 512, 512, 8, 128, 2
    N = (H + 2 * HKV) * D

    def decode(x, qkv_weight, q_norm_weight, k_norm_weight, cache_k, cache_v, start_pos, o_weight):
        return qwen3_attention_kernel(x, qkv_weight, q_norm_weight, k_norm_weight, 1e-6, H, D, HKV,
                                      cache_k, cache_v, start_pos, o_weight)

    args = [_bf16((B, 1, HID)), _bf16((HID, N)), _bf16((D,)), _bf16((D,)), _bf16((B, MAXS, HKV, D)),
            _bf16((B, MAXS, HKV, D)), np.array([7], np.int32), _bf16((H * D, HID))]
    g = NKIPyKernel.trace(decode).specialize(*args)
    plan = lower(g)
    _assert_temps_written_before_read(plan)
    assert plan.kernel_kinds == ["gemm", "head_rope", "decode_attention", "gemm"]
    (step,) = [st for st in plan.steps if st.kind == "head_rope"]
    (launch,) = step.launches(lambda v: 1 << 40)
    a = launch.args
    assert launch.symbol == "nk_head_rope_bf16"
    assert a.tflags == LA.HR_TABLE_F32 and a.pos == 1 << 40
    assert (a.t_row, a.t_rows, a.t_ss, a.S, a.D) == (D // 2, MAXS, 0, 1, D)
    q, k, v = a.t[0], a.t[1], a.t[2]
    # the projection's fp32 partial sums read in place (K ranges of 256: two planes)
    assert (a.plane, a.nplanes) == (B * N, LA.gemv_mfma_split(B, N, HID)[0]) == (B * N, 2)
    for t, heads, col0 in ((q, H, 0), (k, HKV, H * D), (v, HKV, (H + HKV) * D)):
        assert t.H == heads and t.rows == B * heads
        assert (t.x_sb, t.x_sh, t.x_half) == (N, D, D // 2)
        assert t.x == (1 << 40) + 4 * col0
    for t in (q, k):
        assert t.flags == LA.HR_NORM | LA.HR_W | LA.HR_PLANES and np.float32(t.eps) == np.float32(1e-6)
    assert v.flags == LA.HR_COPY | LA.HR_PLANES
    assert (q.o_sb, q.o_sh, q.o_sp) == (H * D, D, 0)
    # k and v go to row pos of their caches (B, MAXS, HKV, D)
    for t in (k, v):
        assert (t.o_sb, t.o_sh, t.o_sp, t.o_rows) == (MAXS * HKV * D, D, HKV * D, MAXS)
    assert launch.grid[0] == -(-B * H // 16) + 2 * -(-B * HKV // 16)
    # prefill: the tables sliced by position instead of taken
    S = 256

    def prefill(x, qkv_weight, q_norm_weight, k_norm_weight, cache_k, cache_v, o_weight):
        return qwen3_attention_kernel(x, qkv_weight, q_norm_weight, k_norm_weight, 1e-6, H, D, HKV,
                                      cache_k, cache_v, None, o_weight)

    g = NKIPyKernel.trace(prefill).specialize(_bf16((B, S, HID)), _bf16((HID, N)), _bf16((D,)), _bf16((D,)),
                                              _bf16((B, MAXS, HKV, D)), _bf16((B, MAXS, HKV, D)),
                                              _bf16((H * D, HID)))
    plan = lower(g)
    _assert_temps_written_before_read(plan)
    kinds = plan.kernel_kinds
    assert kinds.count("head_rope") == 1 and "rmsnorm" not in kinds, kinds
    (step,) = [st for st in plan.steps if st.kind == "head_rope"]
    (launch,) = step.launches(lambda v: 1 << 40)
    a = launch.args
    assert a.pos is None and (a.t_ss, a.S) == (D // 2, S)
    assert (a.t[0].x_ss, a.t[0].x_sb) == (N, S * N)
    # without the pattern the same graph takes the generic steps
    from nkipy_amd.dispatch.patterns import default_patterns
    from nkipy_amd.dispatch.patterns_attention import HeadRopePattern

    pats = [p for p in default_patterns() if not isinstance(p, HeadRopePattern)]
    kinds = lower(g, pats).kernel_kinds
    assert "head_rope" not in kinds and kinds.count("rmsnorm") == 2


def test_lowering_qwen3_prefill_attention_is_one_step():
    """The Qwen3 prefill form (bf16 scores over the whole cache, mask rows
    [:S, :MAXS], bf16 softmax) lowers to one attention step with the score
    cast points and the bf16 softmax as flags: row-max, row-sum and
    weighted-value launches sharing one workspace of two statistics per
    query; keys past S are not read."""
    from nkipy_amd.kernels.qwen3 import prefill_attention_kernel, qwen3_attention_kernel

    B, S, MAXS, Hq, Hkv, D = 1, 2048, 4096, 32, 8, 128
    g = NKIPyKernel.trace(prefill_attention_kernel).specialize(
        _bf16((B, S, Hq, D)), _bf16((B, MAXS, Hkv, D)), _bf16((B, MAXS, Hkv, D)))
    plan = lower(g)
    assert plan.kernel_kinds == ["attention"]
    ((rmax, rsum, smx),) = [st.launches(lambda v: 1 << 40) for st in plan.steps]
    assert [l.symbol for l in (rmax, rsum, smx)] == [
        "nk_attention_rowmax_d128", "nk_attention_rowsum_d128", "nk_attention_causal_d128_sp_xf_bf16"]
    assert rmax.args is smx.args and rsum.args is smx.args
    a = smx.args
    # the divide by sqrt(128) rounds to bf16 as the product by its reciprocal
    # does, for every bf16 score: the kernels multiply
    assert a.flags == LA.ATT_RND_PROD | LA.ATT_RND_SCORE | LA.ATT_SOFTMAX_BF16
    assert np.float32(a.scale) == np.float32(1) / np.float32(np.sqrt(D))
    assert a.S == S and a.causal == 1 and a.rowstat == 1 << 40
    # 512-key chunks: query block qb (128 queries, causal) has ceil((qb + 1) / 4)
    assert (a.ckb, a.nch) == (16, 4)
    assert rmax.grid[0] == rsum.grid[0] == Hq * sum(-(-(qb + 1) // 4) for qb in range(S // 128))
    assert smx.grid[0] == Hq * S // 128
    temps = [b for b in plan.buffers if b.kind == "temp"]
    assert [t.nbytes for t in temps] == [LA.attention_rowstat_bytes(B, S, Hq)]
    # the whole layer: no score matrix, no generic products or softmax
    hid = 512
    kinds = _kinds(qwen3_attention_kernel, _bf16((2, 256, hid)), _bf16((hid, 8 * D)), _bf16((D,)), _bf16((D,)),
                   1e-6, 4, D, 2, _bf16((2, 512, 2, D)), _bf16((2, 512, 2, D)), None, _bf16((4 * D, hid)))
    assert "attention" in kinds and "dot" not in kinds and "softmax" not in kinds, kinds
    # fp32 scores (the Llama form) keep the plain kernel
    from nkipy_amd.kernels import causal_gqa_attention_kernel

    q = _bf16((1, 256, 8, 128))
    g = NKIPyKernel.trace(causal_gqa_attention_kernel).specialize(q, q, q)
    ((launch,),) = [st.launches(lambda v: 1 << 40) for st in lower(g).steps]
    assert launch.symbol == "nk_attention_causal_d128_sp" and launch.args.flags == 0


def test_projection_planes_fold_into_head_prologue():
    """The Qwen3 decode step lowers its QKV projection to the partial-sum
    launch alone, the head prologue adding the planes; a projection whose
    output is also a kernel result keeps its reduction launch."""
    from nkipy_amd.core.trace import NKIPyKernel
    from nkipy_amd.dispatch.lower import lower
    from nkipy_amd.kernels.qwen3 import qwen3_attention_kernel
    from nkipy_amd.kernels.rmsnorm import rmsnorm_kernel

    B, MAXS, H, Hkv, D = 2, 256, 4, 2, 128
    hid = H * D

    def decode(x, qkv_weight, q_norm_weight, k_norm_weight, cache_k, cache_v, start_pos, o_weight):
        return qwen3_attention_kernel(x, qkv_weight, q_norm_weight, k_norm_weight, 1e-6, H, D, Hkv,
                                      cache_k, cache_v, start_pos, o_weight)

    def both(x, qkv_weight, q_norm_weight, k_norm_weight, start_pos):
        from nkipy_amd.core import tensor_apis
        from nkipy_amd.kernels.qwen3 import apply_rotary_emb_kernel, compute_cos_sin_cache

        qkv = np.matmul(x, qkv_weight)
        xq = rmsnorm_kernel(qkv[:, :, :H * D].reshape(B, 1, H, D), q_norm_weight, 1e-6)
        xk = rmsnorm_kernel(qkv[:, :, H * D:(H + Hkv) * D].reshape(B, 1, Hkv, D), k_norm_weight, 1e-6)
        cos, sin = compute_cos_sin_cache(D, MAXS, base=1e6)
        cos = tensor_apis.constant(cos).astype(qkv.dtype)
        sin = tensor_apis.constant(sin).astype(qkv.dtype)
        xq, xk = apply_rotary_emb_kernel(xq, xk, cos[start_pos], sin[start_pos])
        return xq, xk, qkv

    bf = lambda s: dt.to_bf16(np.zeros(s, np.float32))
    g = NKIPyKernel.trace(decode).specialize(bf((B, 1, hid)), bf((hid, (H + 2 * Hkv) * D)), bf(D), bf(D),
                                             bf((B, MAXS, Hkv, D)), bf((B, MAXS, Hkv, D)),
                                             np.array([7], np.int32), bf((H * D, hid)))
    p = lower(g)
    assert p.kernel_kinds[:2] == ["gemm", "head_rope"], p.kernel_kinds
    assert "partial sums to the head prologue" in p.steps[0].desc and "partial-sum planes" in p.steps[1].desc
    assert [l.symbol for l in p.steps[0].launches(lambda v: 1 << 20)] == ["nk_gemv_mfma_nn_bf16_t1"]
    g2 = NKIPyKernel.trace(both).specialize(bf((B, 1, hid)), bf((hid, (H + 2 * Hkv) * D)), bf(D), bf(D),
                                            np.array([7], np.int32))
    p2 = lower(g2)
    assert "head_rope" in p2.kernel_kinds, p2.kernel_kinds
    assert all("partial" not in s.desc for s in p2.steps), [s.desc for s in p2.steps]
