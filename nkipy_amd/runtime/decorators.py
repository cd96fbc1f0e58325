"""``@baremetal_jit`` (reference: nkipy/src/nkipy/runtime/decorators.py:10-64).

Traces the kernel on each call's arguments and runs it through
``baremetal_run_traced_kernel``; loaded kernels are cached by graph hash, so
repeated calls with the same shapes reuse the lowered plan.
"""

import functools

from nkipy_amd.core.compile import trace
from nkipy_amd.runtime.execute import baremetal_run_traced_kernel


def baremetal_jit(kernel_func=None, *, additional_compiler_args="", target=None):
    def decorator(func):
        @functools.wraps(func)
        def wrapper(*args, **kwargs):
            return baremetal_run_traced_kernel(trace(func), *args,
                                               additional_compiler_args=additional_compiler_args,
                                               target=target, **kwargs)

        return wrapper

    if kernel_func is None:
        return decorator
    return decorator(kernel_func)
