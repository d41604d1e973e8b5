"""`axon.candidate_filter` resolves to `enzyme_amd.candidate_filter`."""

import sys as _sys

from enzyme_amd import candidate_filter as _impl

_sys.modules[__name__] = _impl
