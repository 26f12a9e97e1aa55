"""FlyWheel's softmax-attention API on AMD MI355X (gfx950).

A drop-in for the reference package's public surface
(heavyball-research/flywheel-tpu, flywheel_tpu/__init__.py:20-32):
flash_attn_func, flash_attn_varlen_func and flash_attn_with_kvcache, taking
torch tensors (or DLPack-capable arrays) on a HIP device and running the
hand-written kernels of libflywheel_hip.so.  write_kv_cache_pages (one of the
reference's internal exports, flywheel_tpu/__init__.py:39-45) is exported too;
the other internal names that tpu-inference's flywheel backend reads are served
like the reference's (each access warns, FutureWarning): PAGE_SIZE_MULTIPLE is
this backend's page constraint (16), FWD_BLOCKS and NUM_LANES keep the
reference's values (block sizes built from them are accepted), and
merged_cache_heads takes a torch dtype.
"""

import importlib
import warnings

from .decode import flash_attn_with_kvcache
from .page import write_kv_cache_pages
from .prefill import flash_attn_func, flash_attn_varlen_func

__version__ = "0.4.1+mi355x.1"

__all__ = [
    "flash_attn_func",
    "flash_attn_varlen_func",
    "flash_attn_with_kvcache",
    "write_kv_cache_pages",
]


# The names tpu-inference's flywheel backend imports (reference
# flywheel_tpu/__init__.py:35-60); not public API.
INTERNAL_EXPORTS = {
    "PAGE_SIZE_MULTIPLE": "flywheel_tpu.kv_layout",
    "FWD_BLOCKS": "flywheel_tpu.kv_layout",
    "NUM_LANES": "flywheel_tpu.kv_layout",
    "merged_cache_heads": "flywheel_tpu.kv_layout",
}


def __getattr__(name):
    module_name = INTERNAL_EXPORTS.get(name)
    if module_name is None:
        raise AttributeError(f"module 'flywheel_tpu' has no attribute {name!r}")
    warnings.warn(
        f"flywheel_tpu.{name} is internal ({module_name}.{name}): it is exported for"
        " tpu-inference's flywheel backend for now, is not public API and may move or be"
        " removed.", FutureWarning, stacklevel=2)
    return getattr(importlib.import_module(module_name), name)
