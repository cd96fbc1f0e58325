"""Compiled-kernel artefacts on the host (no GPU): the relocatable form of a
lowered plan reproduces, at any 256-byte-aligned buffer addresses, exactly
the argument blocks a fresh lowering produces there; it survives a
save / load round trip; it goes stale when a code object changes."""

import json

import numpy as np
import pytest

from nkipy_amd.core import dtypes as dt
from nkipy_amd.core.trace import NKIPyKernel
from nkipy_amd.dispatch import artifact
from nkipy_amd.dispatch.artifact import RelocatablePlan, _lowered_launches, io_contract
from nkipy_amd.dispatch.lower import lower


def _bf16(shape):
    return dt.to_bf16(np.zeros(shape, np.float32))


def _fp8(shape):
    return np.zeros(shape, np.uint8).view(dt.float8_e4m3fn)


def _kernels():
    from nkipy_amd.kernels import (chunked_linear_attention_kernel, llama_decoder_layer_fp8,
                                   residual_rmsnorm_kernel, softmax_kernel, swiglu_mlp_kernel)

    hid, F, Hq, Hkv, D = 512, 1024, 4, 2, 128
    one = lambda n: np.ones(n, np.float32)

    def generic(cache, upd, idx):
        cache[1:3] = upd
        return np.take(cache, idx, axis=0) * 2.0 + np.sum(cache, axis=1, keepdims=True)[:2]

    return [
        (softmax_kernel, (np.zeros((64, 4096), np.float32),), {}),
        (residual_rmsnorm_kernel, (_bf16((128, 4096)), _bf16((128, 4096)), _bf16((4096,)), 1e-6), {}),
        (swiglu_mlp_kernel, (_bf16((256, 512)), _bf16((512, 1024)), _bf16((512, 1024)), _bf16((1024, 512))), {}),
        (chunked_linear_attention_kernel, (_bf16((1, 2, 1024, 128)),) * 3, {}),
        (llama_decoder_layer_fp8,
         (_bf16((2, 256, hid)), _bf16((hid,)), _fp8(((Hq + 2 * Hkv) * D, hid)), one((Hq + 2 * Hkv) * D),
          _fp8((hid, hid)), one(hid), _bf16((hid,)), _fp8((F, hid)), one(F), _fp8((F, hid)), one(F),
          _fp8((hid, F)), one(hid)), {"n_heads": Hq, "n_kv_heads": Hkv}),
        (generic, (np.zeros((4, 8), np.float32), np.ones((2, 8), np.float32), np.array([0, 3], np.int32)), {}),
    ]


@pytest.mark.parametrize("case", range(6))
def test_relocated_blobs_equal_a_fresh_lowering(case):
    fn, args, kw = _kernels()[case]
    g = NKIPyKernel.trace(fn).specialize(*args, **kw)
    plan = lower(g)
    rp = RelocatablePlan.from_plan(plan, io_contract(g))
    assert len(rp.records) == sum(len(st.launches(lambda v: 1 << 40)) for st in plan.steps)
    rng = np.random.default_rng(case)
    for _ in range(3):
        # arbitrary 256-byte-aligned, non-overlapping buffer addresses
        bases, cur = {}, int(rng.integers(1, 1 << 20)) << 24
        for b in plan.buffers:
            bases[b.index] = cur
            cur += (max(b.nbytes, 16) + 255) // 256 * 256 + int(rng.integers(0, 64)) * 256
        fresh = [bytes(l.args) for _, l in _lowered_launches(plan, bases)]
        assert rp.blobs(bases) == fresh


def test_artifact_round_trip_and_staleness(tmp_path, monkeypatch):
    from nkipy_amd.kernels import llama_decoder_layer_fp8

    fn, args, kw = _kernels()[4]
    g = NKIPyKernel.trace(fn).specialize(*args, **kw)
    plan = lower(g)
    path = tmp_path / "k" / "plan.json"
    assert artifact.write_artifact(plan, g, str(path))
    doc = json.loads(path.read_text())
    assert doc["format"] == artifact.FORMAT and doc["launches"]
    rp = artifact.try_load(str(path), g)
    assert rp is not None and rp.kernel_kinds == plan.kernel_kinds
    bases = {b.index: (1 << 32) + 4096 * b.index * (1 << 12) for b in plan.buffers}
    assert rp.blobs(bases) == RelocatablePlan.from_plan(plan, io_contract(g)).blobs(bases)
    # constants travel as .npy payloads
    consts = [b for b in plan.buffers if b.kind == "const" and b.data is not None]
    for b, lb in zip(consts, [b for b in rp.buffers if b.kind == "const"]):
        assert lb.data.tobytes() == np.ascontiguousarray(dt.numpy_storage(np.ascontiguousarray(b.data))).tobytes()
    # another graph (other I/O contract) does not match
    g2 = NKIPyKernel.trace(fn).specialize(_bf16((1, 256, 512)), *args[1:], **kw)
    assert artifact.try_load(str(path), g2) is None
    # a changed code object makes the artefact stale
    mod = rp.records[0].module
    real = artifact.module_digest
    monkeypatch.setattr(artifact, "module_digest", lambda m: "0" * 16 if m == mod else real(m))
    assert artifact.try_load(str(path), g) is None


def test_unrelocatable_launch_is_not_cached(tmp_path, monkeypatch):
    """A launch whose arguments encode an address other than as an 8-byte
    field (here: the address shifted right by 4) is detected and the
    artefact is written as a description only."""
    from nkipy_amd.dispatch import launchers as LA
    from nkipy_amd.kernels import softmax_kernel

    g = NKIPyKernel.trace(softmax_kernel).specialize(np.zeros((64, 4096), np.float32))
    plan = lower(g)
    real = LA.softmax_rows

    def shifted(x_ptr, y_ptr, *a, **k):
        l = real(x_ptr, y_ptr, *a, **k)
        l.args.rows = x_ptr >> 4  # an address that is not a plain pointer field
        return l

    monkeypatch.setattr(LA, "softmax_rows", shifted)
    path = tmp_path / "plan.json"
    assert not artifact.write_artifact(plan, g, str(path))
    assert json.loads(path.read_text())["relocatable"] is False
    assert artifact.try_load(str(path), g) is None


def test_digest_covers_dtype_table_and_ir(tmp_path, monkeypatch):
    """A change to the dtype table or the IR (both shape the argument blocks)
    makes a saved artefact stale, like a change to the lowering code."""
    from pathlib import Path

    srcs = artifact.lowering_sources()
    names = {(p.parent.name, p.name) for p in srcs}
    assert ("core", "dtypes.py") in names and ("backend", "ir.py") in names
    fn, args, kw = _kernels()[0]
    g = NKIPyKernel.trace(fn).specialize(*args, **kw)
    path = tmp_path / "plan.json"
    assert artifact.write_artifact(lower(g), g, str(path))
    assert artifact.try_load(str(path), g) is not None
    # a copy of the digested files with an edited dtype table
    copies = []
    for i, p in enumerate(srcs):
        c = tmp_path / "src" / str(i) / p.name
        c.parent.mkdir(parents=True)
        data = p.read_bytes()
        if p.name == "dtypes.py" and p.parent.name == "core":
            data += b"\n# edited\n"
        c.write_bytes(data)
        copies.append(Path(c))
    monkeypatch.setattr(artifact, "lowering_sources", lambda: copies)
    monkeypatch.setattr(artifact, "_digest_cache", {})
    assert artifact.try_load(str(path), g) is None


def test_constant_payloads_are_checked_on_load(tmp_path):
    """Payloads are renamed into place after a full write and carry a
    checksum: a truncated or replaced payload is not loaded."""
    fn, args, kw = _kernels()[4]
    g = NKIPyKernel.trace(fn).specialize(*args, **kw)
    path = tmp_path / "plan.json"
    assert artifact.write_artifact(lower(g), g, str(path))
    assert not list(tmp_path.glob("*.tmp"))
    doc = json.loads(path.read_text())
    payloads = [b for b in doc["buffers"] if b["data"]]
    assert payloads and all(len(b["sha256"]) == 64 for b in payloads)
    assert artifact.try_load(str(path), g) is not None
    victim = tmp_path / payloads[0]["data"]
    raw = np.load(victim, allow_pickle=False)
    np.save(victim, raw ^ np.uint8(1), allow_pickle=False)
    assert artifact.try_load(str(path), g) is None
    with pytest.raises(artifact.NotRelocatable):
        RelocatablePlan.load(str(path))
