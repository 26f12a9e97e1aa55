"""FlyWheel's softmax-attention API on AMD MI355X (gfx950).

A drop-in for the reference package's public surface
(heavyball-research/flywheel-tpu, flywheel_tpu/__init__.py:20-32):
flash_attn_func, flash_attn_varlen_func and flash_attn_with_kvcache, taking
torch tensors (or DLPack-capable arrays) on a HIP device and running the
hand-written kernels of libflywheel_hip.so.  write_kv_cache_pages (one of the
reference's internal exports, flywheel_tpu/__init__.py:39-45) is exported too.
"""

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
