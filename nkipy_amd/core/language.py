"""Low-precision dtypes kernels can name (``nl.bfloat16`` and friends).

The reference takes these from neuronxcc (nkipy/src/nkipy/core/language.py:
4-9); here they come from :mod:`nkipy_amd.core.dtypes`, with no compiler
dependency.
"""

from nkipy_amd.core.dtypes import bfloat16, float8_e4m3, float8_e4m3fn, float8_e5m2  # noqa: F401
