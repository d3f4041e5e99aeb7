"""The routing state the reference's tests read from
trnsparse.nki.dispatch (reference trnsparse/nki/dispatch.py:61-81).

`_use_nki()` answers whether calls route to NKI kernels: never on this
build (HAS_NKI is False and set_backend("nki") raises). Which calls run
the HIP kernels is `trnsparse_amd.backend._use_hip()`.
"""

from trnsparse_amd.backend import HAS_NKI, get_backend, set_backend

__all__ = ["HAS_NKI", "set_backend", "get_backend"]


def _use_nki() -> bool:
    return False
