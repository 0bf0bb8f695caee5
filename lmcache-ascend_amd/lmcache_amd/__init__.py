"""MI355X-native replacement for LMCache-Ascend's `c_ops` hot path.

Importing the package installs `lmcache_amd.c_ops` as `lmcache.c_ops` and
`lmcache.non_cuda_equivalents`, the drop-in point the reference uses
(lmcache_ascend/__init__.py:339-367), so upstream LMCache code that calls
`lmc_ops.<name>(...)` reaches the gfx950 kernels.  The import fails when
liblmcache_amd.so has not been built.
"""

from __future__ import annotations

import sys

from .kv_format import KVCacheFormat

__all__ = ["KVCacheFormat", "install", "c_ops"]


def install():
    """Puts this package's c_ops where upstream LMCache imports it from."""
    from . import c_ops

    sys.modules["lmcache.c_ops"] = c_ops
    sys.modules["lmcache.non_cuda_equivalents"] = c_ops
    return c_ops


c_ops = install()
