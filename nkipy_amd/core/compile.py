"""Entry points kept from the reference's ``nkipy.core.compile``
(nkipy/src/nkipy/core/compile.py:22-34,270-309): ``trace``, the
build-directory helpers, ``get_ir`` and ``compile_to_neff``.  There is no
HLO or neuronx-cc step: a traced graph is lowered by :mod:`nkipy_amd.dispatch`
onto precompiled gfx950 kernels, and the "compiled artefact" is that plan in
relocatable form (``nkipy_amd.dispatch.artifact``), loadable with
``DeviceKernel.load_from_neff`` or ``CompiledKernel``.
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


nkipy_compiler_args = ""  # no compiler is invoked; kept for callers that extend it


def get_ir(traced_kernel):
    assert traced_kernel._code is not None, "Kernel must be traced before compilation"
    return traced_kernel._code


def compile_to_neff(trace_kernel, output_dir: str, neff_name: str = "file.neff", target=None,
                    additional_compiler_args: str = "", save_artifacts: bool = False, **_) -> str:
    """Lower the traced kernel and write its plan artefact to
    ``output_dir/neff_name``; returns that path (the reference's signature,
    compile.py:278-309)."""
    from nkipy_amd.dispatch import artifact
    from nkipy_amd.dispatch.lower import lower

    graph = get_ir(trace_kernel)
    path = os.path.join(output_dir, neff_name)
    if not artifact.write_artifact(lower(graph), graph, path):
        raise RuntimeError(f"kernel {graph.name} lowered to launches that cannot be stored as an artefact")
    return path
