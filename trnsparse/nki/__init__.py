"""The reference's backend switch under its own module path
(reference trnsparse/nki/__init__.py:3-5): HAS_NKI, set_backend and
get_backend, the same objects as trnsparse_amd's. HAS_NKI is False on
this build; the HIP kernels are selected with set_backend("hip") or
"auto"."""

from trnsparse_amd.backend import HAS_NKI, get_backend, set_backend

__all__ = ["HAS_NKI", "set_backend", "get_backend"]
