"""`axon.case_gen` resolves to `enzyme_amd.case_gen`."""

import sys as _sys

from enzyme_amd import case_gen as _impl

_sys.modules[__name__] = _impl
