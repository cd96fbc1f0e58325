"""Backend-dispatched operations.

``Op`` keeps the reference's plug-in contract
(nkipy/src/nkipy/core/ops/_registry.py:12-68): implementations register per
backend name with ``@op.impl("<backend>")``; a call dispatches on
``get_backend()`` and raises ``NotImplementedError`` naming the available
backends when the active one has no implementation.  This package registers
``"hip"`` (record IR into the active ``HIPTraceContext``) and, for ops that
must also work outside tracing, ``"cpu"`` (plain NumPy).
"""

from typing import Callable, Dict


class Op:
    def __init__(self, name: str):
        self.name = name
        self._impls: Dict[str, Callable] = {}

    def impl(self, backend: str) -> Callable:
        def decorator(fn: Callable) -> Callable:
            self._impls[backend] = fn
            return fn

        return decorator

    @property
    def backends(self):
        return tuple(self._impls)

    def __call__(self, *args, **kwargs):
        from nkipy_amd.core.backend import get_backend

        backend = get_backend()
        fn = self._impls.get(backend)
        if fn is None:
            available = ", ".join(self._impls) if self._impls else "none"
            raise NotImplementedError(
                f"Operation '{self.name}' not implemented for backend '{backend}'."
                f" Available backends: {available}"
            )
        return fn(*args, **kwargs)

    def __repr__(self) -> str:
        backends = ", ".join(self._impls) if self._impls else "none"
        return f"Op('{self.name}', backends=[{backends}])"
