"""Exact k-nearest-neighbour search by certified exclusion on the AMD Instinct MI355X (gfx950).

The Python surface of the reference package `certex` (certex/__init__.py:48-64): Index, search,
verify, search_stats, trim_pool, auto_width, KeyCache and topk. Every index operation runs through the C API
of libcertex_c.so (include/cuvs/neighbors/certex.h), whose kernels are hand-written HIP for gfx950.
"""

from .attention import KeyCache, topk
from .index import Index, auto_width, row_len, search, search_stats, trim_pool, verify

__version__ = "0.1.0"
__all__ = ["KeyCache", "topk", "Index", "auto_width", "row_len", "search", "search_stats", "trim_pool", "verify",
           "__version__"]
