"""Parity of the HIP kernels with the CPU oracle, through the C ABI (libqvkv.so).

Append, gather and block copy are checked bit for bit; attention within max-abs 2e-3
and relative L2 1e-3 of the oracle's `attend` (f32, the reference's sequential order).
"""

import numpy as np
import pytest

import oracle
from helpers import (F16, MAX_ABS, Q8_0, REL_L2, attn_errors, code_at, decode_pool, normal,
                     random_tables, rng, slots_of)

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def cu32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()


def cu64(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint64).view(np.int64)).cuda()


def cf32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def layout(dtype, G, D, B=16):
    from qubivex_amd import KvLayout

    return KvLayout(dtype, G, D, B)


def new_pool(L, n_blocks, fill=None):
    if fill is None:
        return torch.zeros(n_blocks * L.block_bytes, dtype=torch.uint8, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(fill)
    return torch.randint(0, 256, (n_blocks * L.block_bytes,), dtype=torch.uint8, device="cuda",
                         generator=g)


def is_nan16(h):
    return ((h & 0x7C00) == 0x7C00) & ((h & 0x03FF) != 0)


EDGE_F32 = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e5, 6.1e-5, 6.0e-5,
                     5.96e-8, 2.9802322e-8, 2.9802326e-8, 1e-9, -3e-7, np.inf, -np.inf, np.nan,
                     1.0009765625, 1.00048828125, 1.00146484375, 2049.0, 2051.0, -0.5, 1e-3],
                    np.float32)


@pytest.mark.parametrize("G,D", [(8, 128), (4, 128), (8, 64), (2, 96), (1, 200)])
def test_append_f16_bit_exact(hip, G, D):
    print(f"append f16 G={G} D={D}", flush=True)
    r = rng(100 + G * D)
    L = layout(F16, G, D)
    N, n = 40, 300
    slots = r.choice(N * L.block, n, replace=False).astype(np.uint32)
    k = normal(r, (n, G * D)) * np.float32(r.choice([1e-6, 1e-3, 1.0, 300.0], (n, 1)))
    v = normal(r, (n, G * D))
    k[0, :EDGE_F32.size] = EDGE_F32
    v[1, :EDGE_F32.size] = -EDGE_F32
    pool = new_pool(L, N)
    hip.append(L, pool, N, cf32(k), cf32(v), cu32(slots))
    hip.check()
    dec = decode_pool(pool.cpu().numpy(), L, N)
    want_k = oracle.f16_bits(k).reshape(n, G, D)
    want_v = oracle.f16_bits(v).reshape(n, G, D)
    for i in range(n):
        got = code_at(dec, int(slots[i]), L.block)
        for name, want in (("k", want_k[i]), ("v", want_v[i])):
            g = got[name]
            both_nan = is_nan16(g) & is_nan16(want)
            bad = (g != want) & ~both_nan
            assert not bad.any(), f"row {i} {name}: {g[bad][:4]} vs {want[bad][:4]}"
    # positions never written stay as they were
    written = np.zeros(N * L.block, bool)
    written[slots] = True
    untouched = dec["k"].transpose(0, 2, 1, 3).reshape(N * L.block, G, D)[~written]
    assert not untouched.any()


def q8_case(r, n, G, D):
    """Rows with q8_0 edge groups: zeros, exact .5 ties, a lone outlier, NaN, inf, tiny."""
    k = normal(r, (n, G * D), outliers=0.01)
    v = normal(r, (n, G * D), outliers=0.01)
    grp = k[0].reshape(-1, 32)
    grp[0] = 0.0
    grp[1] = np.linspace(-127, 127, 32).astype(np.float32)
    grp[1, 0], grp[1, 1], grp[1, 2], grp[1, 3] = 127.0, 2.5, -3.5, 0.5  # d = 1: ties
    grp[2, :] = 1e-3
    grp[2, 5] = 40.0
    if grp.shape[0] > 3:
        grp[3, 7] = np.nan
    if grp.shape[0] > 5:
        grp[4] = np.float32(3e-39)  # subnormal amax: 1 / d overflows to inf
        grp[4, 1] = np.float32(-1e-40)
        grp[5] = np.float32(0.5) * np.arange(-16, 16, dtype=np.float32) * np.float32(127 / 15.5)
    gv = v[0].reshape(-1, 32)
    gv[0] = 1e-30  # scale underflows f16 (subnormal / zero)
    gv[1, 3] = np.inf
    if gv.shape[0] > 2:
        gv[2] = -7.0
    return k, v


@pytest.mark.parametrize("G,D", [(8, 128), (4, 64), (2, 256), (3, 96), (5, 128)])
def test_append_q8_0_bit_exact(hip, G, D):
    print(f"append q8_0 G={G} D={D}", flush=True)
    r = rng(200 + G * D)
    L = layout(Q8_0, G, D)
    N, n = 32, 200
    slots = r.choice(N * L.block, n, replace=False).astype(np.uint32)
    k, v = q8_case(r, n, G, D)
    pool = new_pool(L, N)
    hip.append(L, pool, N, cf32(k), cf32(v), cu32(slots))
    hip.check()
    dec = decode_pool(pool.cpu().numpy(), L, N)
    for i in range(n):
        got = code_at(dec, int(slots[i]), L.block)
        for name, x in (("k", k[i]), ("v", v[i])):
            want = oracle.q8_0_quantize(x).reshape(G, D // 32, 34)
            want_scale = want[..., 0].astype(np.uint16) | (want[..., 1].astype(np.uint16) << 8)
            want_q = want[..., 2:].view(np.int8).reshape(G, D)
            gs = got[name + "s"]
            nan_ok = is_nan16(gs) & is_nan16(want_scale)
            assert ((gs == want_scale) | nan_ok).all(), f"row {i} {name} scales"
            assert (got[name] == want_q).all(), f"row {i} {name} values"


@pytest.mark.parametrize("knob", [("append_u", 1), ("append_u", 4), ("append_nt", 1),
                                  ("append_nt", 0), ("append_nts", 0)],
                         ids=lambda kv: f"{kv[0]}={kv[1]}")
@pytest.mark.parametrize("dtype", [F16, Q8_0])
def test_append_builds_are_bit_exact(hip, dtype, knob, knobs):
    """Every append build a knob selects (rows per thread group, cached or non-temporal loads
    and stores) stores the same bytes as the oracle, over 3 layouts each."""
    knobs(*knob)
    for G, D in [(8, 128), (4, 64), (3, 96)]:
        if dtype == F16:
            test_append_f16_bit_exact(hip, G, D)
        else:
            test_append_q8_0_bit_exact(hip, G, D)


def fill_items(hip, L, pool, N, lens, r, outliers=0.0):
    """Appends every position of every item through its table; returns rows and tables."""
    blocks, table_at = random_tables(r, lens, L.block, N)
    ks, vs, ss = [], [], []
    for t, n in enumerate(lens):
        ks.append(normal(r, (n, L.kv_out), outliers))
        vs.append(normal(r, (n, L.kv_out), outliers))
        ss.append(slots_of(blocks, table_at, t, np.arange(n), L.block))
    k, v, s = np.concatenate(ks), np.concatenate(vs), np.concatenate(ss)
    hip.append(L, pool, N, cf32(k), cf32(v), cu32(s))
    hip.check()
    sim = oracle.SimPool(N, L.kv_heads, L.head_dim, L.block, oracle.F16 if L.dtype == F16 else oracle.Q8_0)
    sim.store(k, v, s)
    return blocks, table_at, sim


@pytest.mark.parametrize("dtype,G,D", [(F16, 8, 128), (F16, 4, 64), (Q8_0, 8, 128), (Q8_0, 2, 64),
                                       (Q8_0, 3, 256), (Q8_0, 2, 96), (Q8_0, 1, 160),
                                       (F16, 2, 96)])
def test_gather_bit_exact(hip, dtype, G, D):
    print(f"gather {dtype} G={G} D={D}", flush=True)
    r = rng(300 + G * D)
    L = layout(dtype, G, D)
    lens = [1, 15, 16, 17, 100, 333]
    N = sum((n + 15) // 16 for n in lens) + 7
    pool = new_pool(L, N, fill=5)  # unwritten slots hold garbage: never read
    blocks, table_at, sim = fill_items(hip, L, pool, N, lens, r)
    out_at = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    total = int(sum(lens))
    outs = {}
    for od in (["f32", "f16"] if dtype == F16 else ["f32"]):
        tdt = torch.float32 if od == "f32" else torch.float16
        ok = torch.full((total * L.kv_out,), 7, dtype=tdt, device="cuda")
        ov = torch.full_like(ok, 7)
        hip.gather(L, pool, N, cu32(blocks), cu32(table_at), cu32(lens), cu64(out_at), max(lens),
                   ok, ov, out_dtype=od)
        hip.check()
        outs[od] = (ok.cpu().numpy(), ov.cpu().numpy())
    for t, n in enumerate(lens):
        wk, wv = sim.gather(blocks, table_at, t, n)
        a, b = int(out_at[t]) * L.kv_out, (int(out_at[t]) + n) * L.kv_out
        gk = outs["f32"][0][a:b].reshape(G, n, D)
        gv = outs["f32"][1][a:b].reshape(G, n, D)
        assert np.array_equal(gk.view(np.uint32), wk.view(np.uint32)), f"item {t} keys"
        assert np.array_equal(gv.view(np.uint32), wv.view(np.uint32)), f"item {t} values"
        if "f16" in outs:
            hk = outs["f16"][0][a:b].view(np.uint16).reshape(G, n, D)
            assert np.array_equal(hk, oracle.f16_bits(wk).reshape(G, n, D)), f"item {t} f16 keys"


@pytest.mark.parametrize("dtype,G,D", [(F16, 8, 128), (Q8_0, 3, 160), (Q8_0, 2, 64), (F16, 1, 200)])
def test_block_copy_bytes(hip, dtype, G, D):
    """Blocks of 64 KiB and of sizes that are not a multiple of one workgroup's 1 KiB."""
    L = layout(dtype, G, D)
    N = 64
    pool = new_pool(L, N, fill=11)
    before = pool.cpu().numpy().reshape(N, -1).copy()
    r = rng(12)
    ids = r.permutation(N)
    src, dst = ids[:20].astype(np.uint32), ids[20:40].astype(np.uint32)
    hip.block_copy(L, pool, N, cu32(src), cu32(dst))
    hip.check()
    after = pool.cpu().numpy().reshape(N, -1)
    want = before.copy()
    want[dst] = before[src]
    assert np.array_equal(after, want)


ATTN_CASES = [
    # dtype, H, G, D, context lengths
    (F16, 32, 8, 128, [1, 2, 15, 16, 17, 64, 137, 1000]),
    (F16, 32, 4, 128, [4096, 31, 2048]),
    (F16, 8, 2, 64, [1, 63, 64, 65, 500]),
    (F16, 8, 8, 128, [300, 1]),
    (F16, 16, 1, 128, [700]),  # 16 query heads on one KV head: two head chunks
    (F16, 4, 4, 96, [1, 60, 129]),  # generic kernel
    (F16, 2, 1, 200, [40, 200]),  # generic kernel
    (F16, 4, 2, 256, [100, 513]),
    (Q8_0, 32, 8, 128, [1, 17, 256, 2048]),
    (Q8_0, 32, 4, 128, [5, 1500]),
    (Q8_0, 8, 2, 64, [33, 300]),
    (Q8_0, 4, 2, 256, [90]),
    (Q8_0, 6, 3, 160, [77]),  # generic kernel
    # query groups that are not powers of two (3, 5, 6, 12 heads per KV head)
    (F16, 12, 2, 128, [33, 700]),
    (F16, 24, 2, 128, [129, 16]),
    (Q8_0, 12, 4, 128, [50, 513]),
    (Q8_0, 10, 2, 128, [300]),
    (Q8_0, 24, 2, 64, [95]),
    # 512-767 units (one layer of a decode step): one workgroup per unit, unsplit
    (F16, 32, 8, 128, [(37 * i) % 700 + 1 for i in range(80)]),
    (F16, 16, 1, 128, [(53 * i) % 300 + 1 for i in range(300)]),  # two head chunks
    (Q8_0, 32, 8, 128, [(41 * i) % 700 + 1 for i in range(80)]),
    (Q8_0, 32, 4, 128, [(29 * i) % 500 + 1 for i in range(150)]),
]


@pytest.mark.parametrize("dtype,H,G,D,lens", ATTN_CASES)
def test_attention_within_tolerance(hip, dtype, H, G, D, lens):
    print(f"attention {dtype} H={H} G={G} D={D} lens={lens}", flush=True)
    r = rng(400 + H * G * D + len(lens))
    L = layout(dtype, G, D)
    N = sum((n + 15) // 16 for n in lens) + 3
    pool = new_pool(L, N, fill=9)
    blocks, table_at, sim = fill_items(hip, L, pool, N, lens, r, outliers=0.01 if dtype == Q8_0 else 0)
    q = normal(r, (len(lens), H, D))
    pos = np.array(lens, np.uint32) - 1
    out = torch.full((len(lens) * H * D,), float("nan"), dtype=torch.float32, device="cuda")
    hip.attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32(pos), H, int(pos.max()), out)
    hip.check()
    got = out.cpu().numpy().reshape(len(lens), H, D)
    want = sim.attention(q, H, blocks, table_at, pos)
    max_abs, rel = attn_errors(got, want)
    print(f"  max_abs={max_abs:.2e} rel_l2={rel:.2e}", flush=True)
    assert np.isfinite(got).all()
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)


# Launch switches a caller may set (qvkv_tune knobs, read at each launch) and a few shapes
# each, from ATTN_CASES: every selectable build must meet the same tolerance.
SWITCH_CASES = [ATTN_CASES[i] for i in (0, 1, 8, 9)] + ATTN_CASES[-4:]


@pytest.mark.parametrize("env", [{"attn_waves4_f16": "1"}, {"attn_waves3_q8": "1"},
                                 {"attn_pack": "0"},
                                 {"attn_xcd": "0"}, {"attn_ids_below": "0"},
                                 {"stream_unit_cost": "0"}, {"stream_unit_cost": "40"},
                                 {"attn_stream": "0"}],
                         ids=lambda e: ",".join(f"{k}={v}" for k, v in e.items()))
@pytest.mark.parametrize("dtype,H,G,D,lens", SWITCH_CASES)
def test_attention_launch_switches_stay_within_tolerance(hip, dtype, H, G, D, lens, env,
                                                         knobs):
    for k, v in env.items():
        knobs(k, int(v))
    test_attention_within_tolerance(hip, dtype, H, G, D, lens)


@pytest.mark.parametrize("dtype", [F16, Q8_0])
def test_attention_ignores_nan_in_unwritten_slots(hip, dtype):
    """Slots past each item's last position hold 0xFF bytes: NaN f16 values and NaN q8_0
    scales.  Partial tiles read them; decode and prefill must mask them exactly (q8_0 folds
    the V scale into p with a multiply whose 0 * NaN is 0)."""
    r = rng(410 + (dtype == Q8_0))
    G, D, H = 4, 128, 16
    L = layout(dtype, G, D)
    lens = [1, 7, 17, 250]
    N = sum((n + 15) // 16 for n in lens) + 2
    pool = torch.full((N * L.block_bytes,), 0xFF, dtype=torch.uint8, device="cuda")
    blocks, table_at, sim = fill_items(hip, L, pool, N, lens, r)
    q = normal(r, (len(lens), H, D))
    pos = np.array(lens, np.uint32) - 1
    out = torch.full((len(lens) * H * D,), float("nan"), dtype=torch.float32, device="cuda")
    hip.attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32(pos), H, int(pos.max()), out)
    hip.check()
    got = out.cpu().numpy().reshape(len(lens), H, D)
    assert np.isfinite(got).all()
    e = attn_errors(got, sim.attention(q, H, blocks, table_at, pos))
    assert e[0] <= MAX_ABS and e[1] <= REL_L2, e
    # prefill of every item's last min(n, 9) tokens
    n_tok = np.minimum(np.array(lens), 9).astype(np.uint32)
    pos0 = (np.array(lens) - n_tok).astype(np.uint32)
    q_at = np.concatenate([[0], np.cumsum(n_tok)[:-1]]).astype(np.uint32)
    T = int(n_tok.sum())
    qp = normal(r, (T, H, D))
    outp = torch.full((T * H * D,), float("nan"), dtype=torch.float32, device="cuda")
    hip.prefill_attention(L, pool, N, cf32(qp), cu32(blocks), cu32(table_at), cu32(pos0),
                          cu32(q_at), cu32(n_tok), H, int(max(lens)) - 1, int(n_tok.max()), outp)
    hip.check()
    gp = outp.cpu().numpy().reshape(T, H, D)
    assert np.isfinite(gp).all()
    ta = np.repeat(table_at, n_tok).astype(np.uint32)
    pt = np.concatenate([np.arange(p, p + m) for p, m in zip(pos0, n_tok)]).astype(np.uint32)
    e = attn_errors(gp, sim.attention(qp, H, blocks, ta, pt))
    assert e[0] <= MAX_ABS and e[1] <= REL_L2, e


@pytest.mark.parametrize("split", ["work", "chunks"])
def test_attention_split_context_8k(hip, split, knobs):
    """One long item alone: the launch splits the context (by work, the default, or into
    context chunks) and merges the partials."""
    if split == "chunks":
        knobs("attn_stream", 0)
    r = rng(7)
    L = layout(F16, 4, 128)
    lens = [8192]
    N = 512 + 2
    pool = new_pool(L, N)
    blocks, table_at, sim = fill_items(hip, L, pool, N, lens, r)
    q = normal(r, (1, 32, 128))
    pos = np.array([8191], np.uint32)
    out = torch.zeros(32 * 128, dtype=torch.float32, device="cuda")
    hip.attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32(pos), 32, 8191, out)
    hip.check()
    got = out.cpu().numpy().reshape(1, 32, 128)
    want = sim.attention(q, 32, blocks, table_at, pos)
    max_abs, rel = attn_errors(got, want)
    print(f"  8k split: max_abs={max_abs:.2e} rel_l2={rel:.2e}", flush=True)
    assert max_abs <= MAX_ABS and rel <= REL_L2


@pytest.mark.parametrize("dtype", [F16, Q8_0])
@pytest.mark.parametrize("split", ["work", "chunks"])
def test_attention_split_ragged_batch(hip, dtype, split, knobs):
    """A small ragged batch (one layer of a decode step in model order: 24 items of 1 to
    3000 positions, 8 KV heads, so 192 units): split by work, units are cut across
    workgroup ranges at arbitrary tiles and merged; both split forms against the oracle."""
    if split == "chunks":
        knobs("attn_stream", 0)
    r = rng(71 + (dtype == Q8_0))
    L = layout(dtype, 8, 128)
    lens = [int(x) for x in r.integers(1, 3000, 24)]
    lens[0], lens[1] = 1, 16
    N = sum((n + 15) // 16 for n in lens) + 4
    pool = new_pool(L, N)
    blocks, table_at, sim = fill_items(hip, L, pool, N, lens, r)
    q = normal(r, (len(lens), 32, 128))
    pos = np.array(lens, np.uint32) - 1
    out = torch.full((len(lens) * 32 * 128,), float("nan"), dtype=torch.float32, device="cuda")
    hip.attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32(pos), 32,
                  int(pos.max()), out)
    hip.check()
    got = out.cpu().numpy().reshape(len(lens), 32, 128)
    max_abs, rel = attn_errors(got, sim.attention(q, 32, blocks, table_at, pos))
    print(f"  ragged {dtype} {split}: max_abs={max_abs:.2e} rel_l2={rel:.2e}", flush=True)
    assert max_abs <= MAX_ABS and rel <= REL_L2


def test_attention_special_cases(hip):
    """One position gives v_0 exactly as stored; a zero query gives the mean of v."""
    r = rng(8)
    L = layout(F16, 2, 128)
    lens = [1, 50]
    N = 8
    pool = new_pool(L, N)
    blocks, table_at, sim = fill_items(hip, L, pool, N, lens, r)
    q = normal(r, (2, 4, 128))
    q[1] = 0.0
    pos = np.array([0, 49], np.uint32)
    out = torch.zeros(2 * 4 * 128, dtype=torch.float32, device="cuda")
    hip.attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32(pos), 4, 49, out)
    hip.check()
    got = out.cpu().numpy().reshape(2, 4, 128)
    k0, v0 = sim.gather(blocks, table_at, 0, 1)
    for h in range(4):
        assert np.array_equal(got[0, h], v0[h // 2, 0]), "one position: out = v_0"
    _, v1 = sim.gather(blocks, table_at, 1, 50)
    for h in range(4):
        np.testing.assert_allclose(got[1, h], v1[h // 2].mean(axis=0), atol=1e-5)


def test_decode_attention_host_entry(hip):
    """qvkv_decode_attention: sync rows, then the new rows, then attention, as
    SimDevice::attention (sim.rs:301-436) orders them."""
    from qubivex_amd import KvLayout

    r = rng(9)
    L = KvLayout(F16, 4, 64, 16)
    H = 8
    N = 40
    buf = hip.alloc(N * L.block_bytes)
    pos = np.array([0, 20, 70], np.uint32)
    need = [(int(p) + 16) // 16 for p in pos]
    perm = r.permutation(N).astype(np.uint32)
    blocks = perm[:sum(need)]
    table_at = np.concatenate([[0], np.cumsum(need)[:-1]]).astype(np.uint32)
    # sequence t holds positions 0..pos[t]-1 on the host; all of them are synced now
    sync_rows, sync_to = [], []
    for t, p in enumerate(pos):
        for j in range(int(p)):
            sync_rows.append(normal(r, (2 * L.kv_out,)))
            sync_to.append(int(slots_of(blocks, table_at, t, [j], 16)[0]))
    sync = np.concatenate(sync_rows) if sync_rows else np.zeros(0, np.float32)
    k_new = normal(r, (3, L.kv_out))
    v_new = normal(r, (3, L.kv_out))
    q = normal(r, (3, H, 64))
    got = hip.decode_attention(L, buf, q, H, pos, blocks, table_at, sync, np.array(sync_to, np.uint32),
                               k_new, v_new)
    sim = oracle.SimPool(N, 4, 64, 16, oracle.F16)
    if sync_rows:
        sr = sync.reshape(-1, 2 * L.kv_out)
        sim.store(sr[:, :L.kv_out], sr[:, L.kv_out:], np.array(sync_to, np.uint32))
    new_slots = np.array([slots_of(blocks, table_at, t, [int(p)], 16)[0] for t, p in enumerate(pos)],
                         np.uint32)
    sim.store(k_new, v_new, new_slots)
    want = sim.attention(q, H, blocks, table_at, pos)
    max_abs, rel = attn_errors(got, want)
    assert max_abs <= MAX_ABS and rel <= REL_L2
    tr = hip.transfers()
    assert tr["uploads"] > 0 and tr["downloads"] > 0
    buf.close()


@pytest.mark.parametrize("dtype,D", [(F16, 64), (F16, 128), (Q8_0, 64), (Q8_0, 128)])
def test_index_errors_are_reported_not_faulted(hip, dtype, D):
    """Out-of-range ids come back as ShapeError; the kernels skip them (append, gather and
    decode attention of every form)."""
    from qubivex_amd import ShapeError

    L = layout(dtype, 2, D)
    N = 4
    pool = new_pool(L, N)
    k = cf32(np.ones((1, 2 * D), np.float32))
    hip.append(L, pool, N, k, k, cu32([N * 16 + 3]))
    with pytest.raises(ShapeError):
        hip.check()
    assert int(pool.count_nonzero()) == 0
    # gather through a block id past the pool
    ok = torch.zeros(20 * L.kv_out, dtype=torch.float32, device="cuda")
    ov = torch.zeros_like(ok)
    hip.gather(L, pool, N, cu32([0, 9]), cu32([0]), cu32([20]), cu64([0]), 20, ok, ov)
    with pytest.raises(ShapeError):
        hip.check()
    # gather with a table too short for its length
    hip.gather(L, pool, N, cu32([0]), cu32([0]), cu32([20]), cu64([0]), 20, ok, ov)
    with pytest.raises(ShapeError):
        hip.check()
    q = cf32(np.ones((1, 2, D), np.float32))
    out = torch.zeros(2 * D, dtype=torch.float32, device="cuda")
    hip.attention(L, pool, N, q, cu32([0, 9]), cu32([0]), cu32([20]), 2, 20, out)
    with pytest.raises(ShapeError):
        hip.check()
    # a table too short for the position
    hip.attention(L, pool, N, q, cu32([0]), cu32([0]), cu32([20]), 2, 20, out)
    with pytest.raises(ShapeError):
        hip.check()
    hip.check()  # cleared
    assert int(pool.count_nonzero()) == 0


DOMINANT_CASES = [(F16, 32, 8, 128), (Q8_0, 32, 8, 128), (F16, 16, 4, 64), (Q8_0, 8, 2, 64),
                  (F16, 8, 2, 256), (Q8_0, 8, 2, 256)]


def dominant_items(hip, L, H, r, lens, big):
    """Items of the given lengths whose key at position big[t] is scaled x40, so that one
    score per head sits ~40 (log2 units) away from the rest of its tile; the values stay
    N(0, 1).  Returns the pool, tables, oracle and q."""
    N = sum((n + 15) // 16 for n in lens) + 3
    pool = new_pool(L, N)
    blocks, table_at, sim = fill_items(hip, L, pool, N, lens, r)
    for t, p in enumerate(big):
        k = normal(r, (1, L.kv_out)) * 40.0
        v = normal(r, (1, L.kv_out))
        sl = slots_of(blocks, table_at, t, [p], L.block)
        hip.append(L, pool, N, cf32(k), cf32(v), cu32(sl))
        sim.store(k, v, sl)
    hip.check()
    return N, pool, blocks, table_at, sim, normal(r, (len(lens), H, L.head_dim))


@pytest.mark.parametrize("dtype,H,G,D", DOMINANT_CASES)
def test_attention_with_a_dominant_position(hip, dtype, H, G, D):
    """One position far above the rest of its tile, in each row group of a 16-position
    tile and in later tiles.  The row max must cover all 16 positions of a tile: a max
    over only part of them leaves the dominant probability past the f16 range of the
    P.V operand (inf, then NaN)."""
    print(f"dominant {dtype} H={H} G={G} D={D}", flush=True)
    r = rng(500 + D + G)
    L = layout(dtype, G, D)
    lens = [16, 16, 16, 16, 64, 200, 1]
    big = [3, 7, 11, 15, 60, 100, 0]
    N, pool, blocks, table_at, sim, q = dominant_items(hip, L, H, r, lens, big)
    pos = np.array(lens, np.uint32) - 1
    out = torch.full((len(lens) * H * D,), float("nan"), dtype=torch.float32, device="cuda")
    hip.attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32(pos), H, int(pos.max()), out)
    hip.check()
    got = out.cpu().numpy().reshape(len(lens), H, D)
    want = sim.attention(q, H, blocks, table_at, pos)
    assert np.isfinite(got).all()
    max_abs, rel = attn_errors(got, want)
    print(f"  max_abs={max_abs:.2e} rel_l2={rel:.2e}", flush=True)
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)


POISON_CASES = [(F16, 32, 8, 128), (F16, 8, 2, 64), (F16, 8, 2, 256), (F16, 4, 4, 96),
                (Q8_0, 32, 8, 128), (Q8_0, 8, 2, 64), (Q8_0, 8, 2, 256)]


@pytest.mark.parametrize("dtype,H,G,D", POISON_CASES)
@pytest.mark.parametrize("poison", [float("nan"), float("inf"), float("-inf")])
@pytest.mark.parametrize("where", ["k", "v"])
def test_attention_propagates_nan_and_inf_like_the_reference(hip, dtype, H, G, D, poison, where):
    """One K or V element of one written position is NaN or +-inf (the reference kernel
    harness, crates/qubivex-backend-vulkan/tests/attention_spike.rs:468-486): the outputs
    are NaN exactly where the CPU path's are (q8_0 quantizes the poison first, as the
    reference's quantizer does), and finite outputs stay within tolerance.  Decode attention
    for every form; prefill for q8_0, for NaN, and for the f16 forms that keep the high
    part and residual of q and p apart.  The f16 MFMA prefill at d = 64 and 128 accumulates
    both into one MFMA accumulator, so an infinite f16 key or value (a value past 65504 at
    append) can give NaN there where the reference gives an infinity or a finite value.
    And in every prefill form a non-finite value at one of a segment's own positions
    reaches the segment's earlier tokens as NaN: their probability for it is masked to 0
    and the MFMA's 0 * NaN is NaN.  So the prefill checks keep the poison before the
    segments (item 2's segment is its one poisoned last token)."""
    r = rng(700 + D + G)
    L = layout(dtype, G, D)
    lens = [40, 40, 17]
    N = sum((n + 15) // 16 for n in lens) + 3
    pool = new_pool(L, N)
    blocks, table_at, sim = fill_items(hip, L, pool, N, lens, r)
    # item 0 position 5, KV head 0, d = 3 (and item 2, its last position)
    for t, p in ((0, 5), (2, 16)):
        k = normal(r, (1, L.kv_out))
        v = normal(r, (1, L.kv_out))
        (k if where == "k" else v)[0, 3] = poison
        sl = slots_of(blocks, table_at, t, [p], L.block)
        hip.append(L, pool, N, cf32(k), cf32(v), cu32(sl))
        sim.store(k, v, sl)
    hip.check()
    q = normal(r, (len(lens), H, D))
    pos = np.array(lens, np.uint32) - 1
    out = torch.zeros(len(lens) * H * D, dtype=torch.float32, device="cuda")
    hip.attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32(pos), H, int(pos.max()), out)
    hip.check()
    got = out.cpu().numpy().reshape(len(lens), H, D)
    want = sim.attention(q, H, blocks, table_at, pos)
    assert np.array_equal(np.isnan(got), np.isnan(want)), (np.isnan(got).sum(), np.isnan(want).sum())
    fin = ~np.isnan(want)
    assert np.array_equal(np.isinf(got[fin]), np.isinf(want[fin]))
    ok = np.isfinite(want)
    if ok.any():
        assert np.abs(got[ok] - want[ok]).max() <= MAX_ABS
    if dtype == F16 and D in (64, 128) and not np.isnan(poison):
        return
    # prefill: the last 10 tokens of items 0 and 1, the last token of item 2
    n_tok = np.array([10, 10, 1], np.uint32)
    T = int(n_tok.sum())
    qp = normal(r, (T, H, D))
    outp = torch.zeros(qp.size, dtype=torch.float32, device="cuda")
    pos0 = (np.array(lens) - n_tok).astype(np.uint32)
    q_at = np.concatenate([[0], np.cumsum(n_tok)[:-1]]).astype(np.uint32)

    def prefill():
        hip.prefill_attention(L, pool, N, cf32(qp), cu32(blocks), cu32(table_at), cu32(pos0),
                              cu32(q_at), cu32(n_tok), H, int(max(lens)) - 1, int(n_tok.max()), outp)
        hip.check()

    if dtype == Q8_0 and D == 128 and where == "v" and np.isinf(poison):
        # an infinite value scale: the MFMA prefill reports its range; the f32-scale form
        from qubivex_amd import UnsupportedError
        with pytest.raises(UnsupportedError):
            prefill()
        from qubivex_amd import kv
        with kv.tuned({"prefill_q8_fast": 0}):
            prefill()
    else:
        prefill()
    gotp = outp.cpu().numpy().reshape(T, H, D)
    ta = np.repeat(table_at, n_tok).astype(np.uint32)
    pt = np.concatenate([np.arange(p, p + m) for p, m in zip(pos0, n_tok)]).astype(np.uint32)
    wantp = sim.attention(qp, H, blocks, ta, pt)
    assert np.array_equal(np.isnan(gotp), np.isnan(wantp)), (np.isnan(gotp).sum(), np.isnan(wantp).sum())
    assert np.array_equal(np.isinf(gotp), np.isinf(wantp))
    ok = np.isfinite(wantp)
    if ok.any():
        assert np.abs(gotp[ok] - wantp[ok]).max() <= MAX_ABS


@pytest.mark.parametrize("dtype", [F16, Q8_0])
def test_parity_checks_catch_broken_rules(hip, dtype):
    """Positive controls for the parity checks above (the reference's habit,
    docs/engineering/VULKAN_EXECUTION_AUDIT.md:2499-2513): the same kernel outputs
    compared with an oracle that breaks one rule must fail the check -- a table entry
    swapped with another item's, the causal limit one position short, every tile read from
    the item's first block."""
    r = rng(900 + (dtype == Q8_0))
    L = layout(dtype, 8, 128)
    H = 32
    lens = [300, 130, 47]
    N = sum((n + 15) // 16 for n in lens) + 3
    pool = new_pool(L, N)
    blocks, table_at, sim = fill_items(hip, L, pool, N, lens, r)
    q = normal(r, (len(lens), H, 128))
    pos = np.array(lens, np.uint32) - 1
    out = torch.zeros(len(lens) * H * 128, dtype=torch.float32, device="cuda")
    hip.attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32(pos), H, int(pos.max()), out)
    hip.check()
    got = out.cpu().numpy().reshape(len(lens), H, 128)

    def passes(want):
        e = attn_errors(got, want)
        return e[0] <= MAX_ABS and e[1] <= REL_L2

    assert passes(sim.attention(q, H, blocks, table_at, pos))
    # (a swap inside one item's visible range would not show: attention is a sum over
    # positions, blind to their order; swap a block between two items)
    swapped = blocks.copy()
    swapped[[1, table_at[1] + 1]] = swapped[[table_at[1] + 1, 1]]
    assert not passes(sim.attention(q, H, swapped, table_at, pos))
    assert not passes(sim.attention(q, H, blocks, table_at, pos - 1))
    first = np.repeat(blocks[table_at], [(n + 15) // 16 for n in lens]).astype(np.uint32)
    assert not passes(sim.attention(q, H, first, table_at, pos))
    # gather: bit-exact, so one swapped entry is caught
    total = int(sum(lens))
    out_at = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    ok = torch.zeros(total * L.kv_out, dtype=torch.float32, device="cuda")
    ov = torch.zeros_like(ok)
    hip.gather(L, pool, N, cu32(blocks), cu32(table_at), cu32(lens), cu64(out_at), max(lens), ok, ov)
    hip.check()
    gk = ok.cpu().numpy()[: lens[0] * L.kv_out]
    assert np.array_equal(gk.view(np.uint32), sim.gather(blocks, table_at, 0, lens[0])[0].reshape(-1).view(np.uint32))
    assert not np.array_equal(gk.view(np.uint32), sim.gather(swapped, table_at, 0, lens[0])[0].reshape(-1).view(np.uint32))
