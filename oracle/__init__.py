"""CPU oracle for the paged KV-cache hot path -- TEST INFRASTRUCTURE ONLY.

`oracle.c` restates the reference's CPU arithmetic (f16/q8_0 codecs, `exp`, `softmax`,
`attend`, the simulated device pool's store/gather/attention); `pool_ref.py` restates
the reference's host-side pool logic (free list, block tables, attention plan) and the
prefix-cache index.  Only tests/, `__graft_entry__.smoke()` and bench.py's CPU-baseline
leg may import this package, and only as the checker.  The product path
(`qubivex_amd`) never imports it.
"""
import ctypes
import os

import numpy as np

from .build import LIB, build

F16 = 1
Q8_0 = 2

_lib = None


def lib():
    """The compiled oracle, built on first use if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
        u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
        u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
        sz = ctypes.c_size_t
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16_fixture.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16_fixture.restype = ctypes.c_uint16
        L.orc_exp.argtypes = [ctypes.c_float]
        L.orc_exp.restype = ctypes.c_float
        L.orc_q8_0_quantize.argtypes = [f32p, sz, u8p]
        L.orc_q8_0_dequant.argtypes = [u8p, sz, f32p]
        L.orc_softmax.argtypes = [f32p, sz]
        L.orc_attend.argtypes = [f32p, f32p, f32p, sz, sz, f32p, f32p]
        L.orc_attend_f64.argtypes = [f32p, f32p, f32p, sz, sz, f64p, f64p]
        L.orc_key_word.argtypes = [sz] * 6
        L.orc_key_word.restype = sz
        L.orc_value_word.argtypes = [sz] * 6
        L.orc_value_word.restype = sz
        L.orc_sim_store.argtypes = [f32p, ctypes.c_int, sz, sz, sz, f32p, f32p, u32p, sz]
        L.orc_sim_gather.argtypes = [f32p, sz, sz, sz, u32p, u32p, sz, sz, f32p, f32p]
        L.orc_sim_attention.argtypes = [f32p, sz, sz, sz, sz, u32p, u32p, u32p, sz, f32p,
                                        f32p, ctypes.c_int]
        L.orc_append_rows.argtypes = [f32p, ctypes.c_int, sz, sz, sz, f32p, f32p, u32p, sz,
                                      ctypes.c_int]
        L.orc_max_threads.restype = ctypes.c_int
        u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
        L.orc_f16_encode.argtypes = [f32p, sz, u16p]
        L.orc_f16_decode.argtypes = [u16p, sz, f32p]
        L.orc_exp_vec.argtypes = [f32p, sz, f32p]
        L.orc_reduce_dot.argtypes = [f32p, f32p, sz]
        L.orc_reduce_dot.restype = ctypes.c_float
        L.orc_rms_norm.argtypes = [f32p, f32p, sz, ctypes.c_float]
        L.orc_rope_rotate.argtypes = [f32p, f32p, sz]
        vp = ctypes.c_void_p
        L.orc_prelude.argtypes = [f32p, f32p, f32p, sz, sz, sz, sz, vp, vp, vp, ctypes.c_int,
                                  ctypes.c_float, ctypes.c_int, vp, vp, ctypes.c_float, f32p]
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def f16_to_f32(h):
    return float(lib().orc_f16_to_f32(int(h)))


def f32_to_f16(x):
    return int(lib().orc_f32_to_f16(float(x)))


def f32_to_f16_fixture(x):
    return int(lib().orc_f32_to_f16_fixture(float(x)))


def f16_bits(x):
    """Vector f32 -> f16 bits (uint16), the oracle's RNE narrowing."""
    x = _f32(x).reshape(-1)
    out = np.zeros(x.size, np.uint16)
    lib().orc_f16_encode(x, x.size, out)
    return out


def f16_values(h):
    """Vector f16 bits -> f32 values (the reference's f16_to_f32)."""
    h = np.ascontiguousarray(h, dtype=np.uint16).reshape(-1)
    out = np.zeros(h.size, np.float32)
    lib().orc_f16_decode(h, h.size, out)
    return out


def exp(x):
    return float(lib().orc_exp(float(x)))


def exp_vec(x):
    x = _f32(x).reshape(-1)
    out = np.zeros(x.size, np.float32)
    lib().orc_exp_vec(x, x.size, out)
    return out


def q8_0_quantize(x):
    """x (multiple of 32 values) -> bytes, 34 per 32 values (f16 scale LE, 32 int8)."""
    x = _f32(x).reshape(-1)
    out = np.zeros(x.size // 32 * 34, dtype=np.uint8)
    lib().orc_q8_0_quantize(x, x.size, out)
    return out


def q8_0_dequant(raw, n):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.zeros(n, dtype=np.float32)
    lib().orc_q8_0_dequant(raw, n, out)
    return out


def softmax(x):
    x = _f32(x).copy()
    lib().orc_softmax(x, x.size)
    return x


def attend(q, k, v, pos):
    """math::attend: q [d], k/v [pos+1][d] position-major."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    d = q.size
    out = np.zeros(d, np.float32)
    scores = np.zeros(pos + 1, np.float32)
    lib().orc_attend(q, k, v, d, pos, out, scores)
    return out


def attend_f64(q, k, v, pos):
    q, k, v = _f32(q), _f32(k), _f32(v)
    d = q.size
    out = np.zeros(d, np.float64)
    scores = np.zeros(pos + 1, np.float64)
    lib().orc_attend_f64(q, k, v, d, pos, out, scores)
    return out


def reduce_dot(w, x):
    w, x = _f32(w), _f32(x)
    return float(lib().orc_reduce_dot(w, x, w.size))


def rms_norm(x, w, eps):
    x = _f32(x).copy()
    lib().orc_rms_norm(x, _f32(w), x.size, float(eps))
    return x


def rope_rotate(head, cs):
    head = _f32(head).copy()
    lib().orc_rope_rotate(head, _f32(cs), head.size)
    return head


def prelude(q, k, v, heads, kvh, d, rope, q_bias=None, k_bias=None, v_bias=None, clip=None,
            norm=0, q_norm=None, k_norm=None, eps=1e-6):
    """The host forward pass's prelude (crates/qubivex-arch/src/lib.rs:1258-1292) on copies
    of q [s][heads*d], k, v [s][kvh*d]; rope [s][d].  Returns (q, k, v)."""
    q, k, v = _f32(q).copy(), _f32(k).copy(), _f32(v).copy()
    keep = []

    def ptr(a):
        if a is None:
            return None
        a = _f32(a)
        keep.append(a)
        return a.ctypes.data_as(ctypes.c_void_p)

    s = q.size // (heads * d)
    lib().orc_prelude(q, k, v, s, heads, kvh, d, ptr(q_bias), ptr(k_bias), ptr(v_bias),
                      int(clip is not None), float(clip or 0.0), int(norm), ptr(q_norm),
                      ptr(k_norm), float(eps), _f32(rope))
    return q, k, v


class SimPool:
    """The simulated device pool of the reference (f32 words, reference layout with
    block size B), storing values narrowed through the storage dtype."""

    def __init__(self, n_blocks, kv_heads, head_dim, block, dtype):
        self.G, self.d, self.B, self.dtype = kv_heads, head_dim, block, dtype
        self.kv_out = kv_heads * head_dim
        self.words = np.zeros(n_blocks * 2 * block * self.kv_out, np.float32)

    def store(self, k_rows, v_rows, slots, threads=0):
        k_rows, v_rows, slots = _f32(k_rows), _f32(v_rows), _u32(slots)
        n = slots.size
        assert k_rows.size == n * self.kv_out and v_rows.size == n * self.kv_out
        if threads:
            lib().orc_append_rows(self.words, self.dtype, self.G, self.d, self.B, k_rows,
                                  v_rows, slots, n, threads)
        else:
            lib().orc_sim_store(self.words, self.dtype, self.G, self.d, self.B, k_rows,
                                v_rows, slots, n)

    def gather(self, blocks, table_at, t, n):
        ks = np.zeros(self.G * n * self.d, np.float32)
        vs = np.zeros_like(ks)
        lib().orc_sim_gather(self.words, self.G, self.d, self.B, _u32(blocks), _u32(table_at),
                             t, n, ks, vs)
        return ks.reshape(self.G, n, self.d), vs.reshape(self.G, n, self.d)

    def attention(self, q, heads, blocks, table_at, pos, threads=0):
        pos = _u32(pos)
        q = _f32(q)
        out = np.zeros(pos.size * heads * self.d, np.float32)
        lib().orc_sim_attention(self.words, self.G, self.d, self.B, heads, _u32(blocks),
                                _u32(table_at), pos, pos.size, q, out, threads)
        return out.reshape(pos.size, heads, self.d)

    def copy_block(self, src, dst):
        w = 2 * self.B * self.kv_out
        self.words[dst * w:(dst + 1) * w] = self.words[src * w:(src + 1) * w]
