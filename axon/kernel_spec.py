"""`axon.kernel_spec` resolves to `enzyme_amd.kernel_spec`."""

import sys as _sys

from enzyme_amd import kernel_spec as _impl

_sys.modules[__name__] = _impl
