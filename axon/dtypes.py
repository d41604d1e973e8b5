"""`axon.dtypes` resolves to `enzyme_amd.dtypes`."""

import sys as _sys

from enzyme_amd import dtypes as _impl

_sys.modules[__name__] = _impl
