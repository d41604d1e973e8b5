"""`axon.winner` resolves to `enzyme_amd.winner`."""

import sys as _sys

from enzyme_amd import winner as _impl

_sys.modules[__name__] = _impl
