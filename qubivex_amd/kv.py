"""Host-side mirror of the reference's interface for the paged KV path.

`HipDevice` plays the part of a `DiscreteDevice` backend
(crates/qubivex-compute/src/discrete.rs:433-570): name/describe/usage/transfers,
alloc/write, and the KV entry points.  `KvPool` is the runtime's pool and block tables
(crates/qubivex-runtime/src/discrete.rs:209-290,951-1009) with paged sharing.  Both call
straight into libqvkv.so; device tensors are torch tensors (plumbing: device memory and
streams), and every kernel is the library's HIP code.
"""
import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import F16, F32, Q8_0, check, lib

_DTYPES = {"f16": F16, "q8_0": Q8_0}


def tune(name: str, value: int) -> None:
    """Sets a launch-shape knob (process-wide; see qvkv_tune)."""
    check(lib.qvkv_tune(name.encode(), int(value)))


def tune_get(name: str) -> int:
    v = ctypes.c_int()
    check(lib.qvkv_tune_get(name.encode(), ctypes.byref(v)))
    return v.value


def tune_reset() -> None:
    lib.qvkv_tune_reset()


class tuned:
    """Context manager: knobs set for the block, every knob back to its default after."""

    def __init__(self, knobs: dict):
        self.knobs = dict(knobs)

    def __enter__(self):
        for k, v in self.knobs.items():
            tune(k, v)
        return self

    def __exit__(self, *exc):
        tune_reset()
        return False


@dataclass(frozen=True)
class KvLayout:
    """Storage layout of a pool: dtype ("f16" or "q8_0"), kv_heads, head_dim, block."""

    dtype: str
    kv_heads: int
    head_dim: int
    block: int = 16

    @property
    def code(self):
        return _DTYPES[self.dtype]

    @property
    def c(self):
        return _lib.Layout(self.code, self.kv_heads, self.head_dim, self.block)

    @property
    def kv_out(self):
        return self.kv_heads * self.head_dim

    @property
    def block_bytes(self):
        out = ctypes.c_uint64()
        check(lib.qvkv_block_bytes(ctypes.byref(self.c), ctypes.byref(out)))
        return out.value


class DevicePtr:
    """A raw device address in the shape the bindings take (what `data_ptr()` returns);
    `n`: its element count, for the entry points that take one (numel())."""

    def __init__(self, address: int, n: int = 0):
        self.address = int(address)
        self.n = int(n)

    def data_ptr(self):
        return self.address

    def numel(self):
        return self.n


def _ptr(x):
    """Device pointer of a torch tensor or DevicePtr (or None)."""
    if x is None:
        return None
    return ctypes.c_void_p(x.data_ptr())


def _stream(stream):
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _np(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a, a.ctypes.data_as(ctypes.c_void_p)


class DeviceBuffer:
    """Device memory from HipDevice.alloc: freed by close() or when collected (the
    reference's DeviceBuffer, freed on its last clone, discrete.rs:24-95)."""

    def __init__(self, dev, handle, owned=True):
        self.dev, self.handle, self.owned = dev, handle, owned

    @property
    def ptr(self):
        return lib.qvkv_buf_ptr(self.handle)

    def __len__(self):
        return lib.qvkv_buf_len(self.handle)

    def close(self):
        if self.handle and self.owned:
            lib.qvkv_free(self.handle)
        self.handle = None

    def __del__(self):
        self.close()


class HipDevice:
    """One HIP device through libqvkv (the `DiscreteDevice` trait's surface)."""

    def __init__(self, device: int = 0):
        self.handle = None
        h = ctypes.c_void_p()
        check(lib.qvkv_open(device, ctypes.byref(h)))
        self.handle = h

    # -- DiscreteDevice surface --
    @staticmethod
    def name():
        return "hip"

    def describe(self):
        buf = ctypes.create_string_buffer(256)
        check(lib.qvkv_describe(self.handle, buf, len(buf)))
        return buf.value.decode()

    @staticmethod
    def supports(dtype: str):
        return dtype in _DTYPES

    def usage(self):
        u = _lib.Usage()
        check(lib.qvkv_usage(self.handle, ctypes.byref(u)))
        return {k: getattr(u, k) for k, _ in u._fields_}

    def transfers(self):
        t = _lib.Transfers()
        check(lib.qvkv_transfers(self.handle, ctypes.byref(t)))
        return {k: getattr(t, k) for k, _ in t._fields_}

    def alloc(self, n: int) -> DeviceBuffer:
        h = ctypes.c_void_p()
        check(lib.qvkv_alloc(self.handle, n, ctypes.byref(h)))
        return DeviceBuffer(self, h)

    def write(self, buf: DeviceBuffer, offset: int, data: bytes):
        a, p = _np(np.frombuffer(data, np.uint8), np.uint8)
        check(lib.qvkv_write(self.handle, buf.handle, offset, p, a.nbytes))

    def read(self, buf: DeviceBuffer, offset: int, n: int) -> bytes:
        a = np.zeros(n, np.uint8)
        check(lib.qvkv_read(self.handle, buf.handle, offset, a.ctypes.data_as(ctypes.c_void_p), n))
        return a.tobytes()

    @property
    def stream(self):
        return lib.qvkv_stream(self.handle)

    def timing(self):
        """GPU nanoseconds of the last synchronous (host-memory) call."""
        ns = ctypes.c_uint64()
        check(lib.qvkv_timing(self.handle, ctypes.byref(ns)))
        return ns.value

    def max_arena(self):
        """DiscreteDevice::max_arena: the largest buffer one call can address."""
        n = ctypes.c_uint64()
        check(lib.qvkv_max_arena(self.handle, ctypes.byref(n)))
        return n.value

    def check(self, stream=None):
        """Waits for `stream` and raises ShapeError for an index error a kernel latched
        (UnsupportedError for a q8_0 value scale past the range of the MFMA prefill)."""
        check(lib.qvkv_check(self.handle, _stream(stream)))

    def close(self):
        if self.handle:
            lib.qvkv_close(self.handle)
            self.handle = None

    # -- the hot path on torch device tensors (enqueued on the current torch stream) --
    def append(self, layout: KvLayout, pool, pool_blocks, k, v, slots, stream=None):
        n = slots.numel()
        check(lib.qvkv_append_async(self.handle, ctypes.byref(layout.c), _ptr(pool), pool_blocks,
                                    _ptr(k), _ptr(v), _ptr(slots), n, _stream(stream)))

    def gather(self, layout: KvLayout, pool, pool_blocks, blocks, table_at, lens, out_at,
               max_len, out_k, out_v, out_dtype="f32", stream=None):
        od = F32 if out_dtype == "f32" else F16
        elem = 4 if od == F32 else 2
        out_positions = out_k.numel() * out_k.element_size() // (layout.kv_out * elem)
        check(lib.qvkv_gather_async(self.handle, ctypes.byref(layout.c), _ptr(pool), pool_blocks,
                                    _ptr(blocks), blocks.numel(), _ptr(table_at), _ptr(lens),
                                    _ptr(out_at), lens.numel(), max_len, od, out_positions,
                                    _ptr(out_k), _ptr(out_v), _stream(stream)))

    def append_attention(self, layout: KvLayout, pool, pool_blocks, q, k_new, v_new, blocks,
                         table_at, pos, heads, max_pos, out, stream=None):
        """Stores each item's new key and value rows at its position pos[i], then attends over
        0..pos[i] (the reference's DeviceMoeAttention submission; one launch for f16 pools)."""
        check(lib.qvkv_append_attention_async(self.handle, ctypes.byref(layout.c), _ptr(pool),
                                              pool_blocks, _ptr(q), _ptr(k_new), _ptr(v_new),
                                              _ptr(blocks), blocks.numel(), _ptr(table_at),
                                              _ptr(pos), pos.numel(), heads, max_pos, _ptr(out),
                                              _stream(stream)))

    def attention(self, layout: KvLayout, pool, pool_blocks, q, blocks, table_at, pos, heads,
                  max_pos, out, stream=None):
        check(lib.qvkv_attention_async(self.handle, ctypes.byref(layout.c), _ptr(pool),
                                       pool_blocks, _ptr(q), _ptr(blocks), blocks.numel(),
                                       _ptr(table_at), _ptr(pos), pos.numel(), heads, max_pos,
                                       _ptr(out), _stream(stream)))

    def prefill_attention(self, layout: KvLayout, pool, pool_blocks, q, blocks, table_at, pos0,
                          q_at, n_tok, heads, max_pos, max_tok, out, stream=None):
        """Causal attention of segments of consecutive stored tokens (device tensors):
        token j of segment i is q/out row q_at[i] + j at position pos0[i] + j."""
        q_rows = q.numel() // (heads * layout.head_dim)
        check(lib.qvkv_prefill_attention_async(
            self.handle, ctypes.byref(layout.c), _ptr(pool), pool_blocks, _ptr(q), q_rows,
            _ptr(blocks), blocks.numel(), _ptr(table_at), _ptr(pos0), _ptr(q_at), _ptr(n_tok),
            n_tok.numel(), heads, max_pos, max_tok, _ptr(out), _stream(stream)))

    def block_copy(self, layout: KvLayout, pool, pool_blocks, src, dst, stream=None):
        check(lib.qvkv_block_copy_async(self.handle, ctypes.byref(layout.c), _ptr(pool),
                                        pool_blocks, _ptr(src), _ptr(dst), src.numel(),
                                        _stream(stream)))

    @staticmethod
    def _prelude_struct(heads, norm, clip, eps, ptrs):
        nm = {"none": _lib.NORM_NONE, "full": _lib.NORM_FULL, "per_head": _lib.NORM_PER_HEAD}[norm]
        return _lib.Prelude(heads, nm, int(clip is not None), float(clip or 0.0), float(eps),
                            *[ptrs.get(n) for n in ("q_bias", "k_bias", "v_bias", "q_norm",
                                                    "k_norm", "rope")])

    def prelude(self, layout: KvLayout, heads, q, k, v, rope, norm="none", clip=None, eps=1e-6,
                q_bias=None, k_bias=None, v_bias=None, q_norm=None, k_norm=None, stream=None):
        """The prelude in place on device tensors q [s][heads*d], k, v [s][G*d]."""
        ptrs = {n: (None if t is None else t.data_ptr()) for n, t in
                (("q_bias", q_bias), ("k_bias", k_bias), ("v_bias", v_bias),
                 ("q_norm", q_norm), ("k_norm", k_norm), ("rope", rope))}
        p = self._prelude_struct(heads, norm, clip, eps, ptrs)
        s = q.numel() // (heads * layout.head_dim)
        check(lib.qvkv_prelude_async(self.handle, ctypes.byref(layout.c), ctypes.byref(p),
                                     _ptr(q), _ptr(k), _ptr(v), s, _stream(stream)))

    def prelude_attention(self, layout, buf: DeviceBuffer, heads, q, k, v, rope, pos, blocks,
                          table_at, sync, sync_to, norm="none", clip=None, eps=1e-6,
                          q_bias=None, k_bias=None, v_bias=None, q_norm=None, k_norm=None):
        """One DeviceMoeAttention's KV work from projection outputs (host memory): returns
        (attention out [s][heads][d], k_new, v_new after the prelude)."""
        keep = {}

        def host(name, a):
            if a is None:
                return None
            arr, pp = _np(a, np.float32)
            keep[name] = arr
            return pp.value

        ptrs = {n: host(n, a) for n, a in (("q_bias", q_bias), ("k_bias", k_bias),
                                           ("v_bias", v_bias), ("q_norm", q_norm),
                                           ("k_norm", k_norm), ("rope", rope))}
        p = self._prelude_struct(heads, norm, clip, eps, ptrs)
        q, qp = _np(q, np.float32)
        k, kp = _np(k, np.float32)
        v, vp = _np(v, np.float32)
        pos, pp = _np(pos, np.uint32)
        b, bp = _np(blocks, np.uint32)
        t, tp = _np(table_at, np.uint32)
        sy, syp = _np(sync, np.float32)
        st, stp = _np(sync_to, np.uint32)
        s = pos.size
        out = np.zeros(s * heads * layout.head_dim, np.float32)
        k_new = np.zeros(s * layout.kv_out, np.float32)
        v_new = np.zeros_like(k_new)
        vp_ = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
        check(lib.qvkv_prelude_attention(self.handle, ctypes.byref(layout.c), buf.handle,
                                         ctypes.byref(p), qp, kp, vp, pp, s, bp, b.size, tp, syp,
                                         stp, st.size, vp_(out), vp_(k_new), vp_(v_new)))
        return (out.reshape(s, heads, layout.head_dim), k_new.reshape(s, layout.kv_out),
                v_new.reshape(s, layout.kv_out))

    # -- host-memory forms (synchronous) --
    def append_host(self, layout, buf: DeviceBuffer, k, v, slots):
        k, kp = _np(k, np.float32)
        v, vp = _np(v, np.float32)
        s, sp = _np(slots, np.uint32)
        check(lib.qvkv_append(self.handle, ctypes.byref(layout.c), buf.handle, kp, vp, sp, s.size))

    def gather_host(self, layout, buf: DeviceBuffer, blocks, table_at, lens, out_at,
                    out_positions, out_dtype="f32"):
        od = F32 if out_dtype == "f32" else F16
        npd = np.float32 if od == F32 else np.uint16
        b, bp = _np(blocks, np.uint32)
        t, tp = _np(table_at, np.uint32)
        ln, lp = _np(lens, np.uint32)
        o, op = _np(out_at, np.uint64)
        ok = np.zeros(out_positions * layout.kv_out, npd)
        ov = np.zeros_like(ok)
        check(lib.qvkv_gather(self.handle, ctypes.byref(layout.c), buf.handle, bp, b.size, tp, lp,
                              op, ln.size, od, out_positions, ok.ctypes.data_as(ctypes.c_void_p),
                              ov.ctypes.data_as(ctypes.c_void_p)))
        return ok, ov

    def block_copy_host(self, layout, buf: DeviceBuffer, src, dst):
        s, sp = _np(src, np.uint32)
        d, dp = _np(dst, np.uint32)
        check(lib.qvkv_block_copy(self.handle, ctypes.byref(layout.c), buf.handle, sp, dp, s.size))

    def decode_attention(self, layout, buf: DeviceBuffer, q, heads, pos, blocks, table_at,
                         sync, sync_to, k_new, v_new):
        """One DeviceMoeAttention's KV work (sync rows, new rows, attention), host memory."""
        q, qp = _np(q, np.float32)
        pos, pp = _np(pos, np.uint32)
        b, bp = _np(blocks, np.uint32)
        t, tp = _np(table_at, np.uint32)
        sy, syp = _np(sync, np.float32)
        st, stp = _np(sync_to, np.uint32)
        kn, knp = _np(k_new, np.float32)
        vn, vnp = _np(v_new, np.float32)
        out = np.zeros(pos.size * heads * layout.head_dim, np.float32)
        check(lib.qvkv_decode_attention(self.handle, ctypes.byref(layout.c), buf.handle, qp, heads,
                                        pp, pos.size, bp, b.size, tp, syp, stp, st.size, knp, vnp,
                                        out.ctypes.data_as(ctypes.c_void_p)))
        return out.reshape(pos.size, heads, layout.head_dim)

    def __del__(self):
        self.close()


class PrefixCache:
    """The prefix-cache index (qvkv_prefix_*), the reference's PrefixCache<V>
    (crates/qubivex-kv-cache/src/lib.rs:68-219).  Values may be any Python object (held
    here by id); the C index stores the id.  A paged caller stores pool sequence handles
    and takes a hit with KvPool.fork(value, reuse)."""

    def __init__(self, budget: int):
        h = ctypes.c_void_p()
        check(lib.qvkv_prefix_create(budget, ctypes.byref(h)))
        self.handle = h
        self.budget = budget
        self._values = {}
        self._next = 1

    @staticmethod
    def _scope(scope):
        return None if scope is None else scope.encode()

    def lookup(self, scope, prompt):
        """(value, reuse) of the longest usable prefix, or None."""
        p, pp = _np(prompt, np.uint32)
        val, reuse = ctypes.c_uint64(), ctypes.c_uint32()
        check(lib.qvkv_prefix_lookup(self.handle, self._scope(scope), pp, p.size,
                                     ctypes.byref(val), ctypes.byref(reuse)))
        if reuse.value == 0:
            return None
        return self._values[val.value], reuse.value

    def insert(self, scope, tokens, cost, value):
        t, tp = _np(tokens, np.uint32)
        key = self._next
        self._next += 1
        self._values[key] = value
        kept = ctypes.c_int()
        check(lib.qvkv_prefix_insert(self.handle, self._scope(scope), tp, t.size, cost, key,
                                     ctypes.byref(kept)))
        if not kept.value:
            del self._values[key]
        self._forget_dropped()
        return bool(kept.value)

    def evict_oldest(self):
        ev = ctypes.c_int()
        check(lib.qvkv_prefix_evict_oldest(self.handle, ctypes.byref(ev)))
        self._forget_dropped()
        return bool(ev.value)

    def clear(self):
        check(lib.qvkv_prefix_clear(self.handle))
        self._forget_dropped()

    def cost(self):
        return self.stats()["cost"]

    def stats(self):
        s = _lib.PrefixStats()
        check(lib.qvkv_prefix_stats(self.handle, ctypes.byref(s)))
        return {k: getattr(s, k) for k, _ in s._fields_}

    def _forget_dropped(self):
        self.dropped = getattr(self, "dropped", [])
        n = ctypes.c_uint64()
        check(lib.qvkv_prefix_take_dropped(self.handle, None, 0, ctypes.byref(n)))
        if n.value:
            out = np.zeros(n.value, np.uint64)
            check(lib.qvkv_prefix_take_dropped(self.handle, out.ctypes.data_as(ctypes.c_void_p),
                                               n.value, ctypes.byref(n)))
            for key in out.tolist():
                self.dropped.append(self._values.pop(key))

    def take_dropped(self):
        """Values that left the index since the last call (evicted, replaced, cleared)."""
        d, self.dropped = getattr(self, "dropped", []), []
        return d

    def close(self):
        if self.handle:
            lib.qvkv_prefix_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()


class KvPool:
    """The block pool and block tables (qvkv_pool_*).  dev=None: host-only bookkeeping,
    whose block copies are returned by take_copies() instead of run."""

    def __init__(self, dev, layout: KvLayout, n_blocks: int, n_layers: int):
        self.dev, self.layout, self.n_blocks, self.n_layers = dev, layout, n_blocks, n_layers
        self.handle = None
        h = ctypes.c_void_p()
        check(lib.qvkv_pool_create(dev.handle if dev else None, ctypes.byref(layout.c), n_blocks,
                                   n_layers, ctypes.byref(h)))
        self.handle = h

    @property
    def ptr(self):
        return lib.qvkv_pool_ptr(self.handle)

    @property
    def memory(self):
        """The pool's device memory, for the HipDevice kernel entry points."""
        return DevicePtr(self.ptr)

    @property
    def buffer(self):
        """The pool's device memory as a buffer for the host-memory entry points (owned by
        the pool: not freed by this object)."""
        return DeviceBuffer(self.dev, ctypes.c_void_p(lib.qvkv_pool_buffer(self.handle)),
                            owned=False)

    def stats(self):
        s = _lib.PoolStats()
        check(lib.qvkv_pool_stats(self.handle, ctypes.byref(s)))
        return {k: getattr(s, k) for k, _ in s._fields_}

    def create(self):
        h = ctypes.c_uint32()
        check(lib.qvkv_seq_create(self.handle, ctypes.byref(h)))
        return h.value

    def release(self, seq):
        check(lib.qvkv_seq_release(self.handle, seq))

    def fork(self, parent, positions):
        h = ctypes.c_uint32()
        check(lib.qvkv_seq_fork(self.handle, parent, positions, ctypes.byref(h)))
        return h.value

    def length(self, seq, layer=0):
        n = ctypes.c_uint32()
        check(lib.qvkv_seq_len(self.handle, seq, layer, ctypes.byref(n)))
        return n.value

    def touch(self, seq):
        check(lib.qvkv_seq_touch(self.handle, seq))

    def _copy_stream(self, stream):
        """The stream the pool's copies are ordered after: the given torch stream, else
        torch's current stream (None for a host-only pool)."""
        return None if self.dev is None else _stream(stream)

    def plan_append(self, seqs, counts, layer, stream=None):
        """Slots for counts[i] new positions of seqs[i]; copy-on-write copies run after the
        work queued on `stream` (default: torch's current stream)."""
        s, sp = _np(seqs, np.uint32)
        c, cp = _np(counts, np.uint32)
        out = np.zeros(int(c.sum()), np.uint32)
        check(lib.qvkv_pool_plan_append(self.handle, sp, cp, s.size, layer,
                                        out.ctypes.data_as(ctypes.c_void_p),
                                        self._copy_stream(stream)))
        return out

    def plan_append_layers(self, seqs, counts, layer0, n_layers, stream=None):
        """plan_append on n_layers layers from layer0 at once: slots layer-major, then
        seq-major; one copy-on-write launch for every layer."""
        s, sp = _np(seqs, np.uint32)
        c, cp = _np(counts, np.uint32)
        out = np.zeros(int(c.sum()) * n_layers, np.uint32)
        check(lib.qvkv_pool_plan_append_layers(self.handle, sp, cp, s.size, layer0, n_layers,
                                               out.ctypes.data_as(ctypes.c_void_p),
                                               self._copy_stream(stream)))
        return out

    def plan_attention(self, seqs, pos, epochs, layer, stream=None):
        """attention_plan of one pass (qvkv_pool_plan_attention): returns a dict with
        blocks, table_at, pos, new_slot, sync_to, sync_item, sync_pos."""
        s, sp = _np(seqs, np.uint32)
        p, pp = _np(pos, np.uint32)
        e, ep = _np(epochs, np.uint64)
        cap_b = int(sum(int(x) // self.layout.block + 1 for x in p))
        cap_s = int(p.astype(np.int64).sum())
        blocks = np.zeros(max(cap_b, 1), np.uint32)
        table_at = np.zeros(s.size, np.uint32)
        new_slot = np.zeros(s.size, np.uint32)
        sync_to = np.zeros(max(cap_s, 1), np.uint32)
        sync_item = np.zeros_like(sync_to)
        sync_pos = np.zeros_like(sync_to)
        nt, ns = ctypes.c_uint64(), ctypes.c_uint64()
        vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
        check(lib.qvkv_pool_plan_attention(self.handle, sp, pp, ep, s.size, layer, vp(blocks),
                                           blocks.size, ctypes.byref(nt), vp(table_at),
                                           vp(new_slot), vp(sync_to), vp(sync_item), vp(sync_pos),
                                           sync_to.size, ctypes.byref(ns),
                                           self._copy_stream(stream)))
        n = ns.value
        return {"blocks": blocks[:nt.value], "table_at": table_at, "pos": p, "new_slot": new_slot,
                "sync_to": sync_to[:n], "sync_item": sync_item[:n], "sync_pos": sync_pos[:n]}

    def tables(self, seqs, layer):
        s, sp = _np(seqs, np.uint32)
        cap = sum((self.length(int(x), layer) + self.layout.block - 1) // self.layout.block
                  for x in s)
        blocks = np.zeros(max(cap, 1), np.uint32)
        table_at = np.zeros(s.size, np.uint32)
        pos = np.zeros(s.size, np.uint32)
        n = ctypes.c_uint64()
        check(lib.qvkv_pool_tables(self.handle, sp, s.size, layer,
                                   blocks.ctypes.data_as(ctypes.c_void_p), blocks.size,
                                   ctypes.byref(n), table_at.ctypes.data_as(ctypes.c_void_p),
                                   pos.ctypes.data_as(ctypes.c_void_p)))
        return blocks[:n.value], table_at, pos

    def tables_layers(self, seqs, layer0, n_layers):
        """Every layer's tables in one call: item (l - layer0) * len(seqs) + i."""
        s, sp = _np(seqs, np.uint32)
        cap = sum((self.length(int(x), l) + self.layout.block - 1) // self.layout.block
                  for l in range(layer0, layer0 + n_layers) for x in s)
        blocks = np.zeros(max(cap, 1), np.uint32)
        table_at = np.zeros(s.size * n_layers, np.uint32)
        pos = np.zeros(s.size * n_layers, np.uint32)
        n = ctypes.c_uint64()
        check(lib.qvkv_pool_tables_layers(self.handle, sp, s.size, layer0, n_layers,
                                          blocks.ctypes.data_as(ctypes.c_void_p), blocks.size,
                                          ctypes.byref(n), table_at.ctypes.data_as(ctypes.c_void_p),
                                          pos.ctypes.data_as(ctypes.c_void_p)))
        return blocks[:n.value], table_at, pos

    def device_tables(self, seqs, layer0, n_layers, max_blocks):
        return DeviceTables(self, seqs, layer0, n_layers, max_blocks)

    def evict_lru(self, target_blocks):
        cap = 1 << 16
        out = np.zeros(cap, np.uint32)
        n = ctypes.c_uint32()
        check(lib.qvkv_pool_evict_lru(self.handle, target_blocks,
                                      out.ctypes.data_as(ctypes.c_void_p), cap, ctypes.byref(n)))
        return out[:min(n.value, cap)].tolist()

    def compact(self, seed=0, mode="permute", stream=None):
        """Moves the live blocks to the front (qvkv_pool_compact): mode "permute" (a seeded
        permutation of every live block) or "fill" (blocks past the live count into the
        vacant ids below it, one batch); returns the blocks moved."""
        moved = ctypes.c_uint64()
        m = {"permute": _lib.COMPACT_PERMUTE, "fill": _lib.COMPACT_FILL}[mode]
        check(lib.qvkv_pool_compact(self.handle, m, seed, ctypes.byref(moved),
                                    self._copy_stream(stream)))
        return moved.value

    def refcount(self, block):
        r = ctypes.c_uint32()
        check(lib.qvkv_pool_refcount(self.handle, block, ctypes.byref(r)))
        return r.value

    def take_copies(self):
        n = ctypes.c_uint64()
        check(lib.qvkv_pool_take_copies(self.handle, None, None, 0, ctypes.byref(n)))
        src = np.zeros(n.value, np.uint32)
        dst = np.zeros(n.value, np.uint32)
        if n.value:
            check(lib.qvkv_pool_take_copies(self.handle, src.ctypes.data_as(ctypes.c_void_p),
                                            dst.ctypes.data_as(ctypes.c_void_p), n.value,
                                            ctypes.byref(n)))
        return src, dst

    def take_batches(self):
        """Host-only pools: the block copies issued since the last call, as a list of
        (src, dst) arrays, one per batch (kernel launch)."""
        src, dst = self.take_copies()
        cut = np.nonzero(src == 0xFFFFFFFF)[0]
        out, start = [], 0
        for c in cut:
            out.append((src[start:c], dst[start:c]))
            start = c + 1
        return out

    def close(self):
        if self.handle:
            lib.qvkv_pool_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()


class DeviceTables:
    """Device-resident block tables of a fixed batch (qvkv_tables_*): sync() sends only the
    ids added since the last sync, and the positions; blocks / table_at / pos are device
    arrays for the kernel entry points (item (l - layer0) * len(seqs) + i)."""

    def __init__(self, pool: KvPool, seqs, layer0, n_layers, max_blocks):
        self.pool = pool
        self.handle = None
        s, sp = _np(seqs, np.uint32)
        h = ctypes.c_void_p()
        check(lib.qvkv_tables_create(pool.handle, sp, s.size, layer0, n_layers, max_blocks,
                                     ctypes.byref(h)))
        self.handle = h
        b, t, p, ln = (ctypes.c_void_p() for _ in range(4))
        nt, ni = ctypes.c_uint64(), ctypes.c_uint32()
        check(lib.qvkv_tables_device(h, ctypes.byref(b), ctypes.byref(nt), ctypes.byref(t),
                                     ctypes.byref(p), ctypes.byref(ln), ctypes.byref(ni)))
        self.n_table, self.n_items = nt.value, ni.value
        self.blocks = DevicePtr(b.value, self.n_table)
        self.table_at = DevicePtr(t.value, self.n_items)
        self.pos = DevicePtr(p.value, self.n_items)
        self.lens = DevicePtr(ln.value, self.n_items)
        self.max_pos = 0

    def sync(self, stream=None):
        """Brings the device arrays up to the pool's tables on `stream`; returns max_pos."""
        m = ctypes.c_uint32()
        check(lib.qvkv_tables_sync(self.handle, _stream(stream), ctypes.byref(m)))
        self.max_pos = m.value
        return m.value

    def close(self):
        if self.handle:
            lib.qvkv_tables_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()
