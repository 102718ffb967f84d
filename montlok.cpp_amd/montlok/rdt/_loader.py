"""Load the RDT4quant GPU operators (reference: python/montlok/rdt/_loader.py:153-182).

The reference resolves a prebuilt or JIT-built CPU extension ``montlok._C``.
Here the operators live in ``montlok._C`` (a ctypes module over
``lib/libmlk_hip.so``, built in-tree by ``make -C montlok.cpp_amd``); this
function returns that module. It never falls back to a CPU path.
"""

from __future__ import annotations

from functools import lru_cache


@lru_cache(maxsize=1)
def load_montlok():
    from .. import _C

    _C.library()  # raises when the HIP library is not built
    return _C
