"""Import surface a reference-style kernel needs (CPU only): the annotation
markers of ``nkipy.core.typing`` and the helper ops of
``nkipy.core.tensor_apis``, traced and lowered without a GPU."""

from typing import Optional

import numpy as np
import pytest

import nkipy_amd.core.typing as nt
from nkipy_amd.core import tensor_apis
from nkipy_amd.core.trace import NKIPyKernel
from nkipy_amd.dispatch.lower import lower


def test_typing_markers_are_annotation_types():
    # reference: nkipy/src/nkipy/core/typing.py:5-10
    assert set(nt.__all__) == {"tensor", "mutable_tensor", "mutable", "immutable"}
    opt = Optional[nt.tensor]
    assert nt.tensor in opt.__args__ and type(None) in opt.__args__
    assert issubclass(nt.mutable_tensor, nt.tensor)
    assert nt.mutable[nt.tensor] is nt.mutable and nt.immutable[nt.tensor] is nt.immutable


def test_tensor_apis_exports_match_reference_names():
    # reference: nkipy/src/nkipy/core/tensor_apis.py:5-24
    for name in ("constant", "topk", "rms_norm", "softmax", "conv2d", "conv3d", "zeros", "full"):
        assert hasattr(tensor_apis, name) and name in tensor_apis.__all__


def _annotated_kernel(x, w, start_pos: Optional[nt.tensor] = None, cache: nt.mutable_tensor = None):
    """Reference-style kernel: annotated parameters, helper ops by name."""
    y = tensor_apis.softmax(x, axis=-1)
    if start_pos is not None:
        y = y + start_pos
    return y


def test_annotated_kernel_runs_on_cpu_and_lowers_to_fused_softmax():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((64, 512)).astype(np.float32)
    ref = np.exp(x - x.max(-1, keepdims=True))
    ref /= ref.sum(-1, keepdims=True)
    np.testing.assert_allclose(_annotated_kernel(x, None), ref, rtol=1e-6)  # CPU backend
    plan = lower(NKIPyKernel.trace(_annotated_kernel).specialize(x, np.ones(4, np.float32), None))
    assert plan.kernel_kinds == ["softmax"]


def test_rms_norm_helper_traces_to_the_row_kernel():
    def k(x, w):
        return tensor_apis.rms_norm(x, w, 1e-6)

    x = np.zeros((128, 1024), np.float32)
    w = np.ones(1024, np.float32)
    kinds = lower(NKIPyKernel.trace(k).specialize(x, w)).kernel_kinds
    assert kinds == ["rmsnorm"], kinds


def test_conv_helpers_raise_on_this_backend():
    def k(x, w):
        return tensor_apis.conv2d(x, w)

    with pytest.raises(NotImplementedError):
        NKIPyKernel.trace(k).specialize(np.zeros((1, 1, 4, 4), np.float32), np.zeros((1, 1, 3, 3), np.float32))
