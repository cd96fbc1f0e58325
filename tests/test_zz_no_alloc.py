"""The no-allocation linear-attention entry point against the one that takes
a workspace: bit-identical outputs on two calls in a row (the second
smaller, reusing the device's scratch array), and a clear error for shapes
whose partial states exceed the scratch array."""

import ctypes

import numpy as np
import pytest

from nkipy_amd.core import dtypes as dt
from nkipy_amd.runtime import DeviceTensor
from oracle import numerics as N

pytestmark = pytest.mark.gpu


def _inputs(B, H, T, seed):
    rng = np.random.default_rng(seed)
    return [DeviceTensor.from_numpy(dt.to_bf16(N.bf16_round(rng.standard_normal((B, H, T, 128)) / np.sqrt(128))))
            for _ in range(3)]


def _with_workspace(gpu, q, k, v, B, H, T):
    size = ctypes.c_size_t()
    assert gpu.lib.nkh_linear_attention_workspace_size(B * H, T, ctypes.byref(size)) == 0
    ws = DeviceTensor.empty((max(size.value, 16),), dt.uint8)
    o = DeviceTensor.empty((B, H, T, 128), dt.bfloat16)
    rc = gpu.lib.nkh_linear_attention(q.ptr, k.ptr, v.ptr, o.ptr, B * H, T, ws.ptr, size.value)
    assert rc == 0, gpu.lib.nkh_last_error()
    gpu.sync()
    return dt.numpy_storage(o.numpy()), size.value


def _no_alloc(gpu, q, k, v, B, H, T):
    o = DeviceTensor.empty((B, H, T, 128), dt.bfloat16)
    rc = gpu.lib.nkh_linear_attention_noalloc(q.ptr, k.ptr, v.ptr, o.ptr, B * H, T)
    assert rc == 0, gpu.lib.nkh_last_error()
    gpu.sync()
    return dt.numpy_storage(o.numpy())


def test_no_alloc_matches_workspace_entry_twice(gpu):
    # first call: the linear-attention workload (4 x 16 heads x 8192 tokens,
    # 12.7 MB of partial states); second call: a smaller, differently
    # segmented problem on the same scratch array
    for (B, H, T), seed in (((4, 16, 8192), 1), ((1, 2, 1024), 2)):
        q, k, v = _inputs(B, H, T, seed)
        got = _no_alloc(gpu, q, k, v, B, H, T)
        ref, need = _with_workspace(gpu, q, k, v, B, H, T)
        assert need > 0
        np.testing.assert_array_equal(got, ref)


def test_no_alloc_unsegmented_and_oversized(gpu):
    q, k, v = _inputs(4, 64, 512, 3)  # 256 sequences: no partial states
    np.testing.assert_array_equal(_no_alloc(gpu, q, k, v, 4, 64, 512), _with_workspace(gpu, q, k, v, 4, 64, 512)[0])
    # 3 sequences of 65536 tokens need 25 MB of partial states: rejected
    # before anything is launched
    size = ctypes.c_size_t()
    assert gpu.lib.nkh_linear_attention_workspace_size(3, 65536, ctypes.byref(size)) == 0
    assert size.value > 16 << 20
    big = [DeviceTensor.empty((3, 65536, 128), dt.bfloat16) for _ in range(4)]
    rc = gpu.lib.nkh_linear_attention_noalloc(big[0].ptr, big[1].ptr, big[2].ptr, big[3].ptr, 3, 65536)
    assert rc == 2
    assert b"at most 16777216" in gpu.lib.nkh_last_error()
