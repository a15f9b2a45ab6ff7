"""Backend selection and error types, mirroring the reference's ``omnimem.nsa.backend``.

Reference: src/omnimem/nsa/backend.py:1-59.  There is one backend here, ``"hip"`` (the gfx950
C-ABI library).  The reference's names ``"triton"`` and ``"cuda"`` are accepted as aliases of it
so an existing ``OMNIMEM_NSA_BACKEND`` setting keeps working; any other name raises, as there.
"""
from __future__ import annotations

import os
import threading
from typing import Optional

VALID_BACKENDS = ("hip",)
ALIASES = {"triton": "hip", "cuda": "hip", "hip": "hip"}
ENV_VAR = "OMNIMEM_NSA_BACKEND"

_lock = threading.Lock()
_backend: Optional[str] = None


class NSABackendError(RuntimeError):
    """Raised when the NSA backend cannot serve a request (bad argument, launch failure)."""


class BlockKVBackendError(NSABackendError):
    """Raised when a block-KV cache kernel cannot serve a request."""


def _normalize(name, error: type = NSABackendError, what: str = "invalid NSA backend",
               hint: str = f" (set via {ENV_VAR} or omnimem_amd.backend.set_backend)") -> str:
    key = str(name or "").strip().lower()
    if key not in ALIASES:
        raise error(f"{what} {key!r}; expected one of {tuple(ALIASES)}{hint}")
    return ALIASES[key]


def get_backend() -> str:
    global _backend
    if _backend is None:
        with _lock:
            if _backend is None:
                _backend = _normalize(os.environ.get(ENV_VAR, "hip"))
    return _backend


def set_backend(name: str) -> str:
    global _backend
    name = _normalize(name)
    with _lock:
        _backend = name
    return name


def resolve_backend(name: Optional[str] = None, error: type = ValueError,
                    what: str = "unknown NSA backend") -> str:
    return get_backend() if name is None else _normalize(name, error, what, hint="")


def resolve_block_kv_backend(name: Optional[str] = None) -> str:
    return resolve_backend(name, BlockKVBackendError, "invalid block KV backend")
