"""Native runtime error paths forced from the host (bounds, lifetime, bad code
objects, unknown symbols, argument-size mismatch) and basic device I/O."""

import ctypes
import os

import numpy as np
import pytest

from nkipy_amd.core import dtypes as dt
from nkipy_amd.dispatch import launchers as LA
from nkipy_amd.runtime import DeviceTensor, SpikeError
from nkipy_amd.runtime.hip import HipError, KernelArgumentError

pytestmark = pytest.mark.gpu


def test_roundtrip_dtypes(gpu):
    for arr in [np.arange(10, dtype=np.float32), np.arange(6, dtype=np.int32).reshape(2, 3),
                dt.to_bf16(np.linspace(-2, 2, 9, dtype=np.float32)), np.array([True, False])]:
        t = DeviceTensor.from_numpy(arr, name="t")
        back = t.numpy()
        assert back.dtype == arr.dtype and back.shape == arr.shape
        np.testing.assert_array_equal(dt.numpy_storage(back), dt.numpy_storage(arr))


def test_torch_roundtrip(gpu):
    import torch

    x = torch.randn(4, 5).to(torch.bfloat16)
    t = DeviceTensor.from_torch(x, name="x")
    assert t.dtype == dt.bfloat16
    assert torch.equal(t.torch(), x)
    t.write_from_torch(x * 2)
    assert torch.equal(t.torch(), x * 2)


def test_write_size_mismatch(gpu):
    t = DeviceTensor.from_numpy(np.zeros(4, np.float32))
    with pytest.raises(ValueError):
        t.write_from_numpy(np.zeros(5, np.float32))


def test_out_of_bounds_copy_is_rejected(gpu):
    t = DeviceTensor.from_numpy(np.zeros(4, np.float32))
    buf = np.zeros(8, np.float32)
    with pytest.raises(SpikeError, match="bound"):
        t.tensor_ref.write(buf.ctypes.data, buf.nbytes)
    # past the end through the native bounds check too
    with pytest.raises(SpikeError, match="bound"):
        gpu.h2d(t.ptr + 8, buf.ctypes.data, 16)


def test_use_after_free(gpu):
    t = DeviceTensor.from_numpy(np.zeros(4, np.float32))
    ptr = t.ptr
    t.free()
    with pytest.raises(SpikeError, match="freed"):
        t.numpy()
    with pytest.raises(SpikeError):
        gpu.free(ptr)  # double free rejected natively


def test_unknown_symbol_and_bad_code_object(gpu, tmp_path):
    with pytest.raises(SpikeError):
        gpu.function("rowwise", "nk_does_not_exist")
    bad = tmp_path / "bad.hsaco"
    bad.write_bytes(b"not an elf")
    h = ctypes.c_void_p()
    rc = gpu.lib.nkh_module_load(str(bad).encode(), ctypes.byref(h))
    assert rc != 0
    rc = gpu.lib.nkh_module_load(str(tmp_path / "missing.hsaco").encode(), ctypes.byref(h))
    assert rc != 0 and b"not found" in gpu.lib.nkh_last_error()


def test_kernel_argument_size_mismatch(gpu):
    f = gpu.function("rowwise", "nk_softmax_reg_f32_f32_b256_c2")
    with pytest.raises(KernelArgumentError):
        f.launch((1, 1, 1), (256, 1, 1), b"\x00" * 8)
    with pytest.raises(KernelArgumentError):
        f.launch((1, 1, 1), (1024, 1, 1), LA.SoftmaxArgs())


def test_launch_rejects_bad_shapes_on_host():
    with pytest.raises(LA.LaunchError):
        LA.softmax_rows(0, 0, 0, 10, dt.float32, dt.float32)
    with pytest.raises(LA.LaunchError):
        LA.rmsnorm_rows(0, 0, 4, 16, dt.float32, 1e-6, h_ptr=16)


def test_device_info(gpu):
    info = gpu.device_info()
    assert info["arch"].startswith("gfx950")
    assert info["cu_count"] > 0


def test_reset_runtime_invalidates_loaded_kernels(gpu):
    """After a reset, a kernel loaded before it refuses to run (its code
    objects and temporaries are gone) and a fresh load works."""
    from nkipy_amd.runtime import DeviceKernel
    from nkipy_amd.runtime.hip import get_runtime, reset_runtime

    def kern(a):
        return a * 2.0 + 1.0

    x = np.arange(64, dtype=np.float32).reshape(8, 8)
    dk = DeviceKernel.compile_and_load(kern, x, name="reset_probe")
    ins = {"a": DeviceTensor.from_numpy(x, name="a")}
    np.testing.assert_array_equal(dk(ins)["output0"].numpy(), x * 2 + 1)
    reset_runtime()
    with pytest.raises(SpikeError):
        dk.executor.bind({"a": 1 << 20, "output0": 1 << 21})
    fresh = {"a": DeviceTensor.from_numpy(x, name="a")}
    with pytest.raises(SpikeError):
        dk(fresh)
    dk2 = DeviceKernel.compile_and_load(kern, x, name="reset_probe")
    assert dk2 is not dk and dk2.executor.rt is get_runtime()
    np.testing.assert_array_equal(dk2(fresh)["output0"].numpy(), x * 2 + 1)


def test_save_trace_writes_one_event_per_launch(gpu, tmp_path):
    """save_trace=True profiles one execution (the reference's
    nrt_profile_start / nrt_profile_stop window, spike/src/model.cpp:97-103)
    and writes its trace beside the artefact or at ntff_name."""
    import json

    from nkipy_amd.kernels import residual_rmsnorm_kernel
    from nkipy_amd.runtime import DeviceKernel

    rng = np.random.default_rng(3)
    x = dt.to_bf16(rng.standard_normal((256, 4096)).astype(np.float32))
    w = dt.to_bf16(rng.uniform(0.5, 1.5, 4096).astype(np.float32))
    dk = DeviceKernel.compile_and_load(residual_rmsnorm_kernel, x, x, w, 1e-6, build_dir=str(tmp_path))
    assert repr(dk).startswith("DeviceKernel(")
    ins = {n: DeviceTensor.from_numpy(a, name=n) for n, a in zip(list(dk.input_tensors_info), (x, x, w))}
    plain = dk(ins)
    dest = tmp_path / "prof" / "rms.ntff"
    traced = dk(ins, save_trace=True, ntff_name=str(dest))
    for k in plain:  # the profiled execution computes the same result
        np.testing.assert_array_equal(dt.numpy_storage(traced[k].numpy()), dt.numpy_storage(plain[k].numpy()))
    doc = json.loads(dest.read_text())
    evs = doc["traceEvents"]
    assert len(evs) == len(dk.plan.kernel_kinds) == 1
    assert evs[0]["name"].startswith("nk_rmsnorm") and evs[0]["dur"] > 0 and evs[0]["args"]["bytes"] > 0
    assert doc["otherData"]["steps"] == ["rmsnorm"]
    # default location: beside the compiled artefact
    dk(ins, save_trace=True)
    assert os.path.exists(dk.trace_path())
