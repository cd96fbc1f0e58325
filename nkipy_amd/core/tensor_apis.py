"""Kernel-facing creation helpers (reference: nkipy/src/nkipy/core/tensor_apis.py:3-25)."""

from nkipy_amd.core.ops import (  # noqa: F401
    constant, full, full_like, ones_like, topk, zeros, zeros_like,
)
