"""Entry-point aliases kept from the reference's ``nkipy.core.compile``
(nkipy/src/nkipy/core/compile.py:22-34): ``trace`` and the build-directory
helpers.  There is no HLO or neuronx-cc step: a traced graph is lowered by
:mod:`nkipy_amd.dispatch` onto precompiled gfx950 kernels.
"""

import os

from nkipy_amd.core.trace import NKIPyKernel

trace = NKIPyKernel.trace

_DEFAULT_BUILD_DIR = os.environ.get("NKIPY_BUILD_DIR", "/tmp/build")


def _get_build_dir():
    return _DEFAULT_BUILD_DIR


def _set_build_dir(build_dir):
    global _DEFAULT_BUILD_DIR
    _DEFAULT_BUILD_DIR = build_dir
