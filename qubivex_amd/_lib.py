"""ctypes binding of libqvkv.so (include/qvkv.h).

The library is required: importing this module without a built library raises, so no
caller can silently fall back to anything else.  Build it with
``python qubivex_amd/build.py`` (or ``__graft_entry__.build()``).
"""
import ctypes
import os

from .build import LIB

OK, E_SHAPE, E_UNSUPPORTED, E_OOM, E_DEVICE = 0, 1, 2, 3, 4
F32, F16, Q8_0 = 0, 1, 2


class ComputeError(RuntimeError):
    """A failed call: the reference's ComputeError (crates/qubivex-compute/src/lib.rs:28-83)."""

    code = -1


class ShapeError(ComputeError):
    code = E_SHAPE


class UnsupportedError(ComputeError):
    code = E_UNSUPPORTED


class OutOfDeviceMemory(ComputeError):
    """ComputeError::OutOfDeviceMemory with its fields: bytes requested, in use, capacity."""

    code = E_OOM
    requested = used = capacity = 0


class DeviceError(ComputeError):
    code = E_DEVICE


_BY_CODE = {c.code: c for c in (ShapeError, UnsupportedError, OutOfDeviceMemory, DeviceError)}


class Layout(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("block", ctypes.c_uint32)]


class Usage(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("capacity", "used", "peak", "refused")]


class Transfers(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("uploads", "upload_bytes", "downloads",
                                                "download_bytes", "submissions", "wait_ns",
                                                "timed", "gpu_ns", "stream_waits",
                                                "activations_in", "activations_out",
                                                "transfer_ns", "fence_waits", "submit_ns",
                                                "gpu_busy_ns")]


class PoolStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("bytes", "blocks", "free", "layers", "synced_rows",
                                                "full", "shared_blocks", "cow_copies",
                                                "evicted_blocks", "moved_blocks", "allocated")]


NORM_NONE, NORM_FULL, NORM_PER_HEAD = 0, 1, 2
COMPACT_PERMUTE, COMPACT_FILL = 0, 1


class Prelude(ctypes.Structure):
    _fields_ = [("heads", ctypes.c_uint32), ("norm", ctypes.c_uint32),
                ("has_clip", ctypes.c_uint32), ("clip", ctypes.c_float), ("eps", ctypes.c_float),
                ("q_bias", ctypes.c_void_p), ("k_bias", ctypes.c_void_p),
                ("v_bias", ctypes.c_void_p), ("q_norm", ctypes.c_void_p),
                ("k_norm", ctypes.c_void_p), ("rope", ctypes.c_void_p)]


class PrefixStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("lookups", "hits", "tokens_reused", "inserted",
                                                "evicted", "entries", "cost")]


def _load():
    # torch's HIP runtime first: libqvkv.so then binds the libamdhip64 already in the
    # process.  Loaded the other way round, the process holds two HIP runtimes and the
    # library's sees no device.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    if not os.path.exists(LIB):
        raise ImportError(
            f"libqvkv.so is not built ({LIB}); run `python qubivex_amd/build.py` (or __graft_entry__.build()) first")
    return ctypes.CDLL(LIB)


lib = _load()

_vp, _u32, _u64, _i32, _sz = (ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int,
                              ctypes.c_size_t)
_P = ctypes.POINTER
_LP = _P(Layout)

# name: (restype, argtypes)
SIGNATURES = {
    "qvkv_last_error": (_i32, [ctypes.c_char_p, _sz]),
    "qvkv_last_oom": (_i32, [_P(_u64), _P(_u64), _P(_u64)]),
    "qvkv_open": (_i32, [_i32, _P(_vp)]),
    "qvkv_close": (None, [_vp]),
    "qvkv_describe": (_i32, [_vp, ctypes.c_char_p, _sz]),
    "qvkv_usage": (_i32, [_vp, _P(Usage)]),
    "qvkv_transfers": (_i32, [_vp, _P(Transfers)]),
    "qvkv_stream": (_vp, [_vp]),
    "qvkv_timing": (_i32, [_vp, _P(_u64)]),
    "qvkv_max_arena": (_i32, [_vp, _P(_u64)]),
    "qvkv_tune": (_i32, [ctypes.c_char_p, _i32]),
    "qvkv_tune_get": (_i32, [ctypes.c_char_p, _P(_i32)]),
    "qvkv_tune_reset": (None, []),
    "qvkv_alloc": (_i32, [_vp, _sz, _P(_vp)]),
    "qvkv_free": (None, [_vp]),
    "qvkv_buf_ptr": (_vp, [_vp]),
    "qvkv_buf_len": (_sz, [_vp]),
    "qvkv_write": (_i32, [_vp, _vp, _sz, _vp, _sz]),
    "qvkv_read": (_i32, [_vp, _vp, _sz, _vp, _sz]),
    "qvkv_check": (_i32, [_vp, _vp]),
    "qvkv_block_bytes": (_i32, [_LP, _P(_u64)]),
    "qvkv_append_async": (_i32, [_vp, _LP, _vp, _u64, _vp, _vp, _vp, _u32, _vp]),
    "qvkv_gather_async": (_i32, [_vp, _LP, _vp, _u64, _vp, _u64, _vp, _vp, _vp, _u32, _u32,
                                 _u32, _u64, _vp, _vp, _vp]),
    "qvkv_attention_async": (_i32, [_vp, _LP, _vp, _u64, _vp, _vp, _u64, _vp, _vp, _u32, _u32,
                                    _u32, _vp, _vp]),
    "qvkv_attention_noalloc_async": (_i32, [_vp, _LP, _vp, _u64, _vp, _vp, _u64, _vp, _vp, _u32,
                                            _u32, _u32, _vp, _vp]),
    "qvkv_append_attention_async": (_i32, [_vp, _LP, _vp, _u64, _vp, _vp, _vp, _vp, _u64, _vp,
                                           _vp, _u32, _u32, _u32, _vp, _vp]),
    "qvkv_prefill_attention_async": (_i32, [_vp, _LP, _vp, _u64, _vp, _u64, _vp, _u64, _vp, _vp,
                                            _vp, _vp, _u32, _u32, _u32, _u32, _vp, _vp]),
    "qvkv_block_copy_async": (_i32, [_vp, _LP, _vp, _u64, _vp, _vp, _u32, _vp]),
    "qvkv_append": (_i32, [_vp, _LP, _vp, _vp, _vp, _vp, _u32]),
    "qvkv_gather": (_i32, [_vp, _LP, _vp, _vp, _u64, _vp, _vp, _vp, _u32, _u32, _u64, _vp,
                           _vp]),
    "qvkv_block_copy": (_i32, [_vp, _LP, _vp, _vp, _vp, _u32]),
    "qvkv_decode_attention": (_i32, [_vp, _LP, _vp, _vp, _u32, _vp, _u32, _vp, _u64, _vp, _vp,
                                     _vp, _u32, _vp, _vp, _vp]),
    "qvkv_prelude_async": (_i32, [_vp, _LP, _P(Prelude), _vp, _vp, _vp, _u32, _vp]),
    "qvkv_prelude_attention": (_i32, [_vp, _LP, _vp, _P(Prelude), _vp, _vp, _vp, _vp, _u32, _vp,
                                      _u64, _vp, _vp, _vp, _u32, _vp, _vp, _vp]),
    "qvkv_pool_create": (_i32, [_vp, _LP, _u64, _u32, _P(_vp)]),
    "qvkv_pool_take_copies": (_i32, [_vp, _vp, _vp, _u64, _P(_u64)]),
    "qvkv_pool_destroy": (None, [_vp]),
    "qvkv_pool_ptr": (_vp, [_vp]),
    "qvkv_pool_buffer": (_vp, [_vp]),
    "qvkv_pool_stats": (_i32, [_vp, _P(PoolStats)]),
    "qvkv_seq_create": (_i32, [_vp, _P(_u32)]),
    "qvkv_seq_release": (_i32, [_vp, _u32]),
    "qvkv_seq_fork": (_i32, [_vp, _u32, _u32, _P(_u32)]),
    "qvkv_seq_len": (_i32, [_vp, _u32, _u32, _P(_u32)]),
    "qvkv_seq_touch": (_i32, [_vp, _u32]),
    "qvkv_pool_plan_append": (_i32, [_vp, _vp, _vp, _u32, _u32, _vp, _vp]),
    "qvkv_pool_plan_append_layers": (_i32, [_vp, _vp, _vp, _u32, _u32, _u32, _vp, _vp]),
    "qvkv_pool_tables": (_i32, [_vp, _vp, _u32, _u32, _vp, _u64, _P(_u64), _vp, _vp]),
    "qvkv_pool_plan_attention": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _vp, _u64, _P(_u64), _vp,
                                        _vp, _vp, _vp, _vp, _u64, _P(_u64), _vp]),
    "qvkv_pool_tables_layers": (_i32, [_vp, _vp, _u32, _u32, _u32, _vp, _u64, _P(_u64), _vp, _vp]),
    "qvkv_tables_create": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _P(_vp)]),
    "qvkv_tables_sync": (_i32, [_vp, _vp, _P(_u32)]),
    "qvkv_tables_device": (_i32, [_vp, _P(_vp), _P(_u64), _P(_vp), _P(_vp), _P(_vp), _P(_u32)]),
    "qvkv_tables_destroy": (None, [_vp]),
    "qvkv_pool_evict_lru": (_i32, [_vp, _u64, _vp, _u32, _P(_u32)]),
    "qvkv_pool_compact": (_i32, [_vp, _u32, _u64, _P(_u64), _vp]),
    "qvkv_pool_refcount": (_i32, [_vp, _u32, _P(_u32)]),
    "qvkv_prefix_create": (_i32, [_u64, _P(_vp)]),
    "qvkv_prefix_destroy": (None, [_vp]),
    "qvkv_prefix_lookup": (_i32, [_vp, ctypes.c_char_p, _vp, _u32, _P(_u64), _P(_u32)]),
    "qvkv_prefix_insert": (_i32, [_vp, ctypes.c_char_p, _vp, _u32, _u64, _u64, _P(_i32)]),
    "qvkv_prefix_evict_oldest": (_i32, [_vp, _P(_i32)]),
    "qvkv_prefix_clear": (_i32, [_vp]),
    "qvkv_prefix_stats": (_i32, [_vp, _P(PrefixStats)]),
    "qvkv_prefix_take_dropped": (_i32, [_vp, _vp, _u64, _P(_u64)]),
}

for _name, (_res, _args) in SIGNATURES.items():
    _f = getattr(lib, _name)
    _f.restype = _res
    _f.argtypes = _args


def last_error():
    buf = ctypes.create_string_buffer(1024)
    code = lib.qvkv_last_error(buf, len(buf))
    return code, buf.value.decode(errors="replace")


def check(rc):
    """Raises the ComputeError subclass for a non-zero status."""
    if rc != OK:
        _, msg = last_error()
        exc = _BY_CODE.get(rc, ComputeError)(msg)
        if rc == E_OOM:
            r, u, c = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
            lib.qvkv_last_oom(ctypes.byref(r), ctypes.byref(u), ctypes.byref(c))
            exc.requested, exc.used, exc.capacity = r.value, u.value, c.value
        raise exc
    return rc
