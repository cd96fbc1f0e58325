"""Active trace context and backend selection.

Same contract as the reference's plug-in point
(nkipy/src/nkipy/core/backend/__init__.py:18-58):

* ``tracing(ctx)``           -- install ``ctx`` as the active trace context
* ``get_backend()``          -- ``"cpu"`` with no context, else ``ctx.backend_name``
* ``set_source_location()``  -- forwarded to the active context

A single module-global context: tracing is not re-entrant and not
thread-safe, as in the reference.
"""

from __future__ import annotations

from contextlib import contextmanager
from typing import Optional, Tuple

_active_ctx = None


@contextmanager
def tracing(ctx):
    """Activate ``ctx`` (an object with a ``backend_name``) while the block runs."""
    global _active_ctx
    _active_ctx = ctx
    try:
        yield ctx
    finally:
        _active_ctx = None


def get_backend() -> str:
    if _active_ctx is not None:
        return _active_ctx.backend_name
    return "cpu"


def get_active_context():
    return _active_ctx


def set_source_location(location: Optional[Tuple[str, int]]) -> None:
    if _active_ctx is not None:
        _active_ctx.set_source_location(location)
