"""Parameter annotations kernels may import as ``nt`` (reference:
nkipy/src/nkipy/core/typing.py:5-10, which re-exports the NKI compiler's
``tensor`` / ``mutable_tensor`` / ``mutable`` / ``immutable``).

Here they are plain marker classes with no compiler behind them.  Tracing
binds arguments by position and name and never reads annotations, so a
kernel annotated ``start_pos: Optional[nt.tensor]`` or
``cache: nt.mutable_tensor`` traces exactly as without the annotation; a
parameter is treated as mutated because the kernel writes to it, not because
of its annotation.  ``nt.mutable[...]`` / ``nt.immutable[...]`` subscript to
themselves, so parametrised spellings stay valid annotations.
"""

from __future__ import annotations

__all__ = ["tensor", "mutable_tensor", "mutable", "immutable"]


class _Marker(type):
    def __repr__(cls):
        return f"nt.{cls.__name__}"

    def __getitem__(cls, _item):
        return cls


class tensor(metaclass=_Marker):
    """A tensor parameter (an ndarray on the CPU, a traced tensor under trace)."""


class mutable_tensor(tensor):
    """A tensor parameter the kernel writes in place."""


class mutable(metaclass=_Marker):
    """Qualifier for a parameter the kernel writes in place."""


class immutable(metaclass=_Marker):
    """Qualifier for a parameter the kernel only reads."""
