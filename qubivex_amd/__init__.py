"""qubivex_amd: the paged KV-cache hot path of qubivex, native to one MI355X (gfx950).

libqvkv.so holds the HIP kernels (append with f16 / q8_0 quantize-on-write, block-table
gather, MFMA paged decode attention, batched block copy), the C ABI of include/qvkv.h,
and the host pool manager (block tables, prefix sharing with copy-on-write, LRU
eviction, compaction).  This package is its Python binding.
"""
from ._lib import (ComputeError, DeviceError, OutOfDeviceMemory, ShapeError,  # noqa: F401
                   UnsupportedError)
from .kv import DeviceBuffer, DevicePtr, HipDevice, KvLayout, KvPool, PrefixCache  # noqa: F401
