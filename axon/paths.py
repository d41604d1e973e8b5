"""`axon.paths` resolves to `enzyme_amd.paths`."""

import sys as _sys

from enzyme_amd import paths as _impl

_sys.modules[__name__] = _impl
