"""`axon.bench_runner` resolves to `enzyme_amd.bench_runner`."""

import sys as _sys

from enzyme_amd import bench_runner as _impl

_sys.modules[__name__] = _impl
