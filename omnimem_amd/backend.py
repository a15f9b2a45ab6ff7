"""Backend selection for the NSA operators.

The reference lets a process pick one of two kernel backends, from ``OMNIMEM_NSA_BACKEND`` or
``set_backend`` (src/omnimem/nsa/backend.py:9-59), and raises ``NSABackendError`` /
``BlockKVBackendError`` for names it does not know.  This build has exactly one backend, the
gfx950 HIP library, so "selecting" it only validates a name: ``"hip"``, and the reference's
``"cuda"`` and ``"triton"`` as other spellings of it, so an environment written for the
reference keeps working.  Every accepted name resolves to ``"hip"``.

The environment variable is checked once, on the first ``get_backend`` call.  There is no
mutable selection to protect, so no lock is needed.
"""
from __future__ import annotations

import os
from typing import Optional

ENV_VAR = "OMNIMEM_NSA_BACKEND"
BACKEND = "hip"
VALID_BACKENDS = (BACKEND,)
_SPELLINGS = (BACKEND, "cuda", "triton")


class NSABackendError(RuntimeError):
    """An NSA operator cannot serve a request (bad argument, unsupported shape, launch failure)."""


class BlockKVBackendError(NSABackendError):
    """A block-KV cache operator cannot serve a request."""


def _accept(name, error: type, context: str) -> str:
    spelled = "" if name is None else str(name).strip().lower()
    if spelled not in _SPELLINGS:
        raise error(f"{context}: backend {spelled!r} is not available; this build runs the "
                    f"gfx950 HIP library, named by any of {_SPELLINGS}")
    return BACKEND


_env_checked = False


def get_backend() -> str:
    """The active backend: always ``"hip"``.  Raises if ``OMNIMEM_NSA_BACKEND`` names another."""
    global _env_checked
    if not _env_checked:
        value = os.environ.get(ENV_VAR)
        if value is not None:
            _accept(value, NSABackendError, ENV_VAR)
        _env_checked = True
    return BACKEND


def set_backend(name: str) -> str:
    """Check that ``name`` selects this build's backend; returns ``"hip"``."""
    return _accept(name, NSABackendError, "set_backend")


def resolve_backend(name: Optional[str] = None, error: type = ValueError,
                    what: str = "unknown NSA backend") -> str:
    """An explicit per-call backend name, checked (``error`` if unknown); None means active."""
    return get_backend() if name is None else _accept(name, error, what)


def resolve_block_kv_backend(name: Optional[str] = None) -> str:
    """As ``resolve_backend`` for the block-KV kernels, raising ``BlockKVBackendError``."""
    return resolve_backend(name, BlockKVBackendError, "block KV backend")
