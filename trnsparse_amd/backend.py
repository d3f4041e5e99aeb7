"""Backend selection: the seam between the public ops and the HIP kernels.

Mirrors the reference's routing state (trnsparse/nki/dispatch.py:61-81):
a module-level backend name set with `set_backend` and read with
`get_backend`, resolved per call by `_use_hip()` (the reference's
`_use_nki()`).

Backends
- "hip":     hand-written gfx950 kernels through libtrnsparse_hip.so.
- "pytorch": the reference's in-file torch semantics (trnsparse/ops.py),
             selected explicitly by the caller.
- "auto":    "hip" whenever a ROCm GPU is visible, else "pytorch" (the
             reference resolves "auto" to its accelerator the same way,
             dispatch.py:76-81).
- "nki":     accepted for API compatibility; raises (no Neuron here).

There is no silent fallback: when the "hip" backend is in effect and the
library cannot be loaded or a kernel fails, the op raises RuntimeError.
"""

from __future__ import annotations

import functools

import torch

HAS_NKI = False
_backend = "auto"


@functools.lru_cache(maxsize=None)
def _gpu_visible() -> bool:
    return bool(torch.cuda.is_available()) and torch.version.hip is not None


def _lib_loads() -> bool:
    try:
        from .hip import _lib

        _lib.load()
        return True
    except Exception:
        return False


def has_hip() -> bool:
    """True when a ROCm GPU is visible and libtrnsparse_hip.so loads."""
    return _gpu_visible() and _lib_loads()


def set_backend(backend: str) -> None:
    global _backend
    assert backend in ("auto", "pytorch", "hip", "nki")
    if backend == "nki":
        raise RuntimeError("NKI backend requires Neuron hardware; this build targets MI355X (use 'hip')")
    if backend == "hip" and not _gpu_visible():
        raise RuntimeError("HIP backend requires a visible ROCm GPU")
    _backend = backend


def get_backend() -> str:
    return _backend


def _use_hip() -> bool:
    if _backend == "hip":
        return True
    if _backend == "pytorch":
        return False
    return _gpu_visible()

