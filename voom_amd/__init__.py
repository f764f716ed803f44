"""voom_amd -- MI355X-native paged-KV path of the vOOM runtime.

Decode attention through a page table (GQA and absorbed-MLA), the byte-plane
spill codec and page reload run as hand-written gfx950 HIP kernels in
libvoom_hip.so (C ABI in include/voom_hip.h); this package is the Python host
layer that mirrors the reference's PagedKVCache API.
"""

from ._build import LIB_PATH  # noqa: F401

__all__ = ["LIB_PATH"]
