"""Shared test helpers: seeded inputs, block tables, and an independent numpy decoder of
the pool's storage layout (the layout contract of include/qvkv.h / kernels.hip)."""
import numpy as np

F16, Q8_0 = "f16", "q8_0"


def rng(seed):
    return np.random.default_rng(seed)


def normal(r, shape, outliers=0.0, scale=8.0):
    """N(0,1) float32; a fraction `outliers` of elements multiplied by `scale`."""
    x = r.standard_normal(shape, dtype=np.float32)
    if outliers:
        m = r.random(shape) < outliers
        x[m] *= scale
    return x


def kperm(d, D):
    """Byte of logical value d in a stored q8_0 key row."""
    d = np.asarray(d)
    return ((d & 31) >> 3) * (D >> 2) + (d >> 5) * 8 + (d & 7)


def vperm(d, D):
    """Byte of logical value d in a stored q8_0 value row."""
    d = np.asarray(d)
    return ((d & 31) >> 1) * (D >> 4) + 2 * (d >> 5) + (d & 1)


def decode_pool(raw, layout, n_blocks):
    """Pool bytes -> per-block codes in logical order.

    f16: {"k": uint16 [N][G][B][D], "v": ...}
    q8_0: {"k": int8 [N][G][B][D], "ks": uint16 [N][G][B][D/32], "v": ..., "vs": ...}
    """
    G, D, B = layout.kv_heads, layout.head_dim, layout.block
    raw = np.asarray(raw, np.uint8).reshape(n_blocks, layout.block_bytes)
    rows = G * B
    if layout.dtype == F16:
        k = raw[:, :rows * D * 2].copy().view(np.uint16).reshape(n_blocks, G, B, D)
        v = raw[:, rows * D * 2:].copy().view(np.uint16).reshape(n_blocks, G, B, D)
        return {"k": k, "v": v}
    q, s = rows * D, rows * (D // 32) * 2
    kq = raw[:, :q].view(np.int8).reshape(n_blocks, G, B, D)
    ks = raw[:, q:q + s].copy().view(np.uint16).reshape(n_blocks, G, B, D // 32)
    vq = raw[:, q + s:2 * q + s].view(np.int8).reshape(n_blocks, G, B, D)
    vs = raw[:, 2 * q + s:].copy().view(np.uint16).reshape(n_blocks, G, B, D // 32)
    d = np.arange(D)
    return {"k": kq[..., kperm(d, D)], "ks": ks, "v": vq[..., vperm(d, D)], "vs": vs}


def code_at(dec, slot, B):
    """The stored codes of pool position `slot` (block*B + offset), per head."""
    b, o = slot // B, slot % B
    return {name: arr[b, :, o] for name, arr in dec.items()}


def random_tables(r, lens, B, n_blocks):
    """Block tables for items of the given lengths, drawn from a shuffled pool."""
    need = [(int(n) + B - 1) // B for n in lens]
    assert sum(need) <= n_blocks
    ids = r.permutation(n_blocks).astype(np.uint32)
    blocks = ids[:sum(need)]
    table_at = np.concatenate([[0], np.cumsum(need)[:-1]]).astype(np.uint32)
    return blocks, table_at


def slots_of(blocks, table_at, t, positions, B):
    positions = np.asarray(positions, np.int64)
    return (blocks[table_at[t] + positions // B].astype(np.int64) * B + positions % B).astype(
        np.uint32)


def attn_errors(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    diff = got - want
    max_abs = float(np.max(np.abs(diff))) if diff.size else 0.0
    rel_l2 = float(np.linalg.norm(diff) / max(np.linalg.norm(want), 1e-30))
    return max_abs, rel_l2


# The north star's attention tolerance: max-abs 2e-3 and relative L2 1e-3 (fp32 accumulation).
MAX_ABS = 2e-3
REL_L2 = 1e-3
