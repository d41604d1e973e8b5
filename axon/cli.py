"""`axon.cli` resolves to `enzyme_amd.cli`."""

import sys as _sys

from enzyme_amd import cli as _impl

_sys.modules[__name__] = _impl
