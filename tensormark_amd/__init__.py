"""MI355X-native token sampler: TensorMark's sampling path as HIP kernels for gfx950.

The C ABI is include/tmsample_hip.h, implemented by libtmsample_hip.so (built
by ``python -m tensormark_amd.build``).  ``tensormark_amd.sampler`` is the
Python host side over it.
"""
from .sampler import (  # noqa: F401
    EXPORTS,
    HISTORY_DTYPE,
    Opts,
    RowParams,
    ROW_DTYPE,
    Sampler,
    load_library,
    make_history,
    make_params,
)

__all__ = ["EXPORTS", "HISTORY_DTYPE", "Opts", "RowParams", "ROW_DTYPE", "Sampler", "load_library",
           "make_history", "make_params"]
