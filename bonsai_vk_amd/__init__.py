"""bonsai_vk_amd - MI355X (gfx950) KV-cache path of bonsai-vk behind a C ABI (include/bkv.h).

The compute runs in libbkv.so (hand-written HIP). This package is the Python host mirror used by
tests and bench.py: device memory comes from torch, everything else goes through the C ABI."""
from ._lib import BKV_F16, BKV_Q8_0, BkvCacheDesc, BkvError, lib  # noqa: F401
from .cache import KvGeom, KvCache  # noqa: F401
