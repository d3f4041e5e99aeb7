"""trnsparse — the reference's import name for this MI355X build.

Callers and tests of the reference write `import trnsparse`
(reference trnsparse/__init__.py:10-33). This package is that name over
`trnsparse_amd`: the same objects (formats, ops, solvers, the backend
switch), so `trnsparse.spmv is trnsparse_amd.spmv`, and the submodules
`trnsparse.formats`, `trnsparse.ops`, `trnsparse.iterative` and
`trnsparse.nki` resolve to this build's modules. Nothing here computes.
"""

import sys as _sys

import trnsparse_amd as _impl
from trnsparse_amd import *  # noqa: F401,F403  (the public names, __all__ below)
from trnsparse_amd import __version__, formats, iterative, ops  # noqa: F401

from . import nki  # noqa: F401  (HAS_NKI, set_backend, get_backend)

# `import trnsparse.formats` / `from trnsparse.ops import spmv` reach the same modules
for _name in ("formats", "ops", "iterative"):
    _sys.modules[f"{__name__}.{_name}"] = getattr(_impl, _name)

__all__ = list(_impl.__all__)
