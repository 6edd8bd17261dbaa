"""rmda_moe: MI355X-native MoE feed-forward path of R-MDA's teacher layer.

The product is the C-ABI library librmda_moe.so (include/rmda_moe.h, sources
in r-mda_amd/csrc).  This package is its Python mirror for tests and the
benchmark: ctypes bindings, the benchmark configurations and the
synthetic-input generator.
"""
from . import configs
from ._lib import LIB_PATH, NONE, NO_SLOT, header_functions, lib

__all__ = ["configs", "lib", "LIB_PATH", "NONE", "NO_SLOT", "header_functions", "Context", "MoeError"]


def __getattr__(name):
    # torch is imported lazily so host-only helpers work without it
    if name in ("Context", "MoeError", "workspace_bytes", "workspace_layout", "ws_views", "packed_bytes"):
        from . import api
        return getattr(api, name)
    raise AttributeError(name)
