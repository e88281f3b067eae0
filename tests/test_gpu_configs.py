"""The BASELINE.json configurations at their real shapes, through the C ABI.

cfg1: small Llama-like KV, one sequence: prefill 512, then 128 decode steps of append +
      gather + attention, every step checked against the oracle.
cfg2: Llama-3-8B-like batched decode (32 sequences, contexts U[256, 4096]).
cfg3: q8_0 KV, 64 sequences x 2048 with 1 % x8 outliers.
cfg4: prefix sharing with copy-on-write, LRU eviction of 25 % and seeded compaction.
(cfg5, 128 x 8k, is bench.py's workload; its parity is sampled in test_cfg5_sampled.)

At full size the checks are size-independent properties (gather(append(x)) == f16(x) for
every position of every item; unchanged reads across COW, eviction and compaction; finite
outputs) plus oracle attention on sampled items.
"""
import numpy as np
import pytest

import oracle
from helpers import MAX_ABS, REL_L2, attn_errors, random_tables, slots_of

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def t32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()


def t64(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint64).view(np.int64)).cuda()


def oracle_attention(k, v, q, n):
    """attend per head from gathered logical values: k, v [G][n][d]; q [H][d]."""
    H, d = q.shape
    G = k.shape[0]
    out = np.zeros((H, d), np.float32)
    for h in range(H):
        g = h // (H // G)
        out[h] = oracle.attend(q[h], k[g, :n], v[g, :n], n - 1)
    return out


def test_cfg1_small_llama_decode_loop(hip):
    """16 layers, 8 KV heads, d 64, 32 query heads, block 16, f16: prefill-append 512
    positions, then 128 x (append 1, gather, attention), each against the oracle."""
    from qubivex_amd import KvLayout

    print("cfg1", flush=True)
    L, G, D, H, B = 16, 8, 64, 32, 16
    layout = KvLayout("f16", G, D, B)
    r = np.random.default_rng(101)
    cap = 512 + 128
    N = L * (cap // B) + 37
    blocks, table_at = random_tables(r, [cap] * L, B, N)  # seeded shuffled free list
    pool = torch.zeros(N * layout.block_bytes, dtype=torch.uint8, device="cuda")
    sim = oracle.SimPool(N, G, D, B, oracle.F16)
    d_blocks, d_tab = t32(blocks), t32(table_at)

    def append_positions(p0, n):
        k = r.standard_normal((L * n, G * D), dtype=np.float32)
        v = r.standard_normal((L * n, G * D), dtype=np.float32)
        slots = np.concatenate([slots_of(blocks, table_at, l, np.arange(p0, p0 + n), B)
                                for l in range(L)])
        hip.append(layout, pool, N, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), t32(slots))
        sim.store(k, v, slots)

    append_positions(0, 512)
    worst = (0.0, 0.0)
    for step in range(128):
        p = 512 + step
        append_positions(p, 1)
        n = p + 1
        lens = np.full(L, n, np.uint32)
        out_at = (np.arange(L) * n).astype(np.uint64)
        ok = torch.empty(L * n * G * D, dtype=torch.float32, device="cuda")
        ov = torch.empty_like(ok)
        hip.gather(layout, pool, N, d_blocks, d_tab, t32(lens), t64(out_at), n, ok, ov)
        q = r.standard_normal((L, H, D), dtype=np.float32)
        out = torch.empty(L * H * D, dtype=torch.float32, device="cuda")
        pos = np.full(L, p, np.uint32)
        hip.attention(layout, pool, N, torch.from_numpy(q).cuda(), d_blocks, d_tab, t32(pos), H, p, out)
        hip.check()
        gk = ok.cpu().numpy().reshape(L, G, n, D)
        gv = ov.cpu().numpy().reshape(L, G, n, D)
        if step % 16 == 0 or step == 127:
            for l in range(L):
                wk, wv = sim.gather(blocks, table_at, l, n)
                assert np.array_equal(gk[l], wk) and np.array_equal(gv[l], wv), (step, l)
        want = sim.attention(q, H, blocks, table_at, pos)
        e = attn_errors(out.cpu().numpy().reshape(L, H, D), want)
        worst = (max(worst[0], e[0]), max(worst[1], e[1]))
    print(f"  cfg1 worst max_abs={worst[0]:.2e} rel_l2={worst[1]:.2e}", flush=True)
    assert worst[0] <= MAX_ABS and worst[1] <= REL_L2


def fill_layerwise(hip, layout, pool, N, blocks, table_at, items_per_layer, L, lens, gen,
                   outliers=0.0):
    """Appends positions 0..lens[s]-1 of every (layer, sequence) item, layer by layer, from
    a seeded torch generator; returns the f32 source rows per layer, [sum(lens)][kv_out]."""
    B = layout.block
    src = []
    for l in range(L):
        slots = np.concatenate([slots_of(blocks, table_at, l * items_per_layer + s,
                                         np.arange(lens[s]), B) for s in range(items_per_layer)])
        k = torch.randn((slots.size, layout.kv_out), generator=gen, device="cuda")
        v = torch.randn((slots.size, layout.kv_out), generator=gen, device="cuda")
        if outliers:
            for x in (k, v):
                m = torch.rand(x.shape, generator=gen, device="cuda") < outliers
                x[m] *= 8.0
        hip.append(layout, pool, N, k, v, t32(slots))
        src.append((k, v))
    hip.check()
    return src


def check_gather_f16(hip, layout, pool, N, blocks, table_at, lens, L, S, src):
    """gather(append(x)) == f16(x) for every position of every item (torch's RNE cast as
    the independent reference for this size-independent property)."""
    G, D = layout.kv_heads, layout.head_dim
    for l in range(L):
        items = l * S + np.arange(S)
        ln = np.asarray(lens, np.uint32)
        out_at = np.concatenate([[0], np.cumsum(ln[:-1], dtype=np.uint64)]).astype(np.uint64)
        tot = int(ln.sum())
        ok = torch.empty(tot * G * D, dtype=torch.float16, device="cuda")
        ov = torch.empty_like(ok)
        hip.gather(layout, pool, N, t32(blocks), t32(table_at[items]), t32(ln), t64(out_at),
                   int(ln.max()), ok, ov, out_dtype="f16")
        hip.check()
        k, v = src[l]
        for s in range(S):
            n = int(ln[s])
            a = int(out_at[s])
            gk = ok[a * G * D:(a + n) * G * D].view(G, n, D)
            want = k[a:a + n].view(n, G, D).permute(1, 0, 2).half()
            assert torch.equal(gk.view(torch.int16), want.contiguous().view(torch.int16)), (l, s)
            gv = ov[a * G * D:(a + n) * G * D].view(G, n, D)
            wv = v[a:a + n].view(n, G, D).permute(1, 0, 2).half()
            assert torch.equal(gv.view(torch.int16), wv.contiguous().view(torch.int16)), (l, s)


def test_cfg2_batched_decode_llama3_8b(hip):
    from qubivex_amd import KvLayout

    print("cfg2", flush=True)
    L, G, D, H, B, S = 32, 8, 128, 32, 16, 32
    layout = KvLayout("f16", G, D, B)
    r = np.random.default_rng(202)
    ctx = r.integers(256, 4097, S)
    lens_items = np.tile(ctx, L)
    need = int(sum((int(c) + B - 1) // B for c in lens_items))
    N = int(np.ceil(1.25 * need))
    blocks, table_at = random_tables(r, lens_items, B, N)
    pool = torch.zeros(N * layout.block_bytes, dtype=torch.uint8, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(202)
    # positions 0..ctx-2 were prefilled; the decode step appends ctx-1
    src = fill_layerwise(hip, layout, pool, N, blocks, table_at, S, L, ctx - 1, gen)
    pos = (lens_items - 1).astype(np.uint32)
    new_slots = np.array([slots_of(blocks, table_at, t, [int(pos[t])], B)[0] for t in range(S * L)],
                         np.uint32)
    kn = torch.randn((S * L, G * D), generator=gen, device="cuda")
    vn = torch.randn((S * L, G * D), generator=gen, device="cuda")
    hip.append(layout, pool, N, kn, vn, t32(new_slots))
    q = torch.randn((S * L, H, D), generator=gen, device="cuda")
    out = torch.empty((S * L, H, D), device="cuda")
    hip.attention(layout, pool, N, q, t32(blocks), t32(table_at), t32(pos), H, int(pos.max()), out)
    hip.check()
    assert torch.isfinite(out).all()
    # every position of every item, bit for bit (sources: prefill rows + the new row)
    full = []
    for l in range(L):
        k, v = src[l]
        ks, vs, off = [], [], 0
        for s in range(S):
            n = int(ctx[s]) - 1
            ks += [k[off:off + n], kn[l * S + s:l * S + s + 1]]
            vs += [v[off:off + n], vn[l * S + s:l * S + s + 1]]
            off += n
        full.append((torch.cat(ks), torch.cat(vs)))
    check_gather_f16(hip, layout, pool, N, blocks, table_at, ctx, L, S, full)
    # oracle attention on sampled items, from the verified gathered values
    for t in r.choice(S * L, 6, replace=False):
        n = int(pos[t]) + 1
        items = np.array([t])
        ok = torch.empty(n * G * D, dtype=torch.float32, device="cuda")
        ov = torch.empty_like(ok)
        hip.gather(layout, pool, N, t32(blocks), t32(table_at[items]), t32([n]), t64([0]), n, ok, ov)
        hip.check()
        want = oracle_attention(ok.cpu().numpy().reshape(G, n, D), ov.cpu().numpy().reshape(G, n, D),
                                q[t].cpu().numpy(), n)
        e = attn_errors(out[t].cpu().numpy(), want)
        assert e[0] <= MAX_ABS and e[1] <= REL_L2, (t, e)


def test_cfg3_q8_0_decode(hip):
    from qubivex_amd import KvLayout

    print("cfg3", flush=True)
    L, G, D, H, B, S, CTX = 32, 8, 128, 32, 16, 64, 2048
    layout = KvLayout("q8_0", G, D, B)
    r = np.random.default_rng(303)
    lens_items = np.full(S * L, CTX)
    N = S * L * (CTX // B) + 11
    blocks, table_at = random_tables(r, lens_items, B, N)
    pool = torch.zeros(N * layout.block_bytes, dtype=torch.uint8, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(303)
    src = fill_layerwise(hip, layout, pool, N, blocks, table_at, S, L, np.full(S, CTX - 1), gen,
                         outliers=0.01)
    pos = np.full(S * L, CTX - 1, np.uint32)
    new_slots = np.array([slots_of(blocks, table_at, t, [CTX - 1], B)[0] for t in range(S * L)], np.uint32)
    kn = torch.randn((S * L, G * D), generator=gen, device="cuda")
    vn = torch.randn((S * L, G * D), generator=gen, device="cuda")
    hip.append(layout, pool, N, kn, vn, t32(new_slots))
    q = torch.randn((S * L, H, D), generator=gen, device="cuda")
    out = torch.empty((S * L, H, D), device="cuda")
    hip.attention(layout, pool, N, q, t32(blocks), t32(table_at), t32(pos), H, CTX - 1, out)
    hip.check()
    assert torch.isfinite(out).all()
    for t in r.choice(S * L, 4, replace=False):
        l, s = divmod(int(t), S)
        ok = torch.empty(CTX * G * D, dtype=torch.float32, device="cuda")
        ov = torch.empty_like(ok)
        hip.gather(layout, pool, N, t32(blocks), t32(table_at[[t]]), t32([CTX]), t64([0]), CTX, ok, ov)
        hip.check()
        k, v = src[l]
        rows_k = torch.cat([k[s * (CTX - 1):(s + 1) * (CTX - 1)], kn[t:t + 1]]).cpu().numpy()
        rows_v = torch.cat([v[s * (CTX - 1):(s + 1) * (CTX - 1)], vn[t:t + 1]]).cpu().numpy()
        wk = oracle.q8_0_dequant(oracle.q8_0_quantize(rows_k), rows_k.size).reshape(CTX, G, D)
        wv = oracle.q8_0_dequant(oracle.q8_0_quantize(rows_v), rows_v.size).reshape(CTX, G, D)
        gk = ok.cpu().numpy().reshape(G, CTX, D)
        gv = ov.cpu().numpy().reshape(G, CTX, D)
        assert np.array_equal(gk, wk.transpose(1, 0, 2)), t
        assert np.array_equal(gv, wv.transpose(1, 0, 2)), t
        want = oracle_attention(gk, gv, q[t].cpu().numpy(), CTX)
        e = attn_errors(out[t].cpu().numpy(), want)
        print(f"  cfg3 item {t}: max_abs={e[0]:.2e} rel_l2={e[1]:.2e}", flush=True)
        assert e[0] <= MAX_ABS and e[1] <= REL_L2, (t, e)


def test_cfg4_prefix_sharing_cow_eviction_compaction(hip):
    from qubivex_amd import KvLayout, KvPool

    print("cfg4", flush=True)
    L, G, D, B, S = 32, 8, 128, 16, 64
    PREFIX, DIV = 2047, 256
    layout = KvLayout("f16", G, D, B)
    N = 48000
    pool = KvPool(hip, layout, N, L)
    mem = pool.memory
    gen = torch.Generator(device="cuda").manual_seed(404)
    r = np.random.default_rng(404)

    def append(seqs, counts, l):
        slots = pool.plan_append(seqs, counts, l)
        k = torch.randn((slots.size, layout.kv_out), generator=gen, device="cuda")
        v = torch.randn((slots.size, layout.kv_out), generator=gen, device="cuda")
        hip.append(layout, mem, N, k, v, t32(slots))
        return k, v

    def read(seq, l):
        blocks, table_at, pos = pool.tables([seq], l)
        n = int(pos[0]) + 1
        ok = torch.empty(n * G * D, dtype=torch.float16, device="cuda")
        ov = torch.empty_like(ok)
        hip.gather(layout, mem, N, t32(blocks), t32(table_at), t32([n]), t64([0]), n, ok, ov,
                   out_dtype="f16")
        hip.check()
        return ok.view(G, n, D), ov.view(G, n, D)

    def as_heads(x):
        return x.view(-1, G, D).permute(1, 0, 2).half().contiguous()

    # Grow the library's staging buffer first, so no allocation inside the copy-on-write
    # calls below waits for the device: the copies must be ordered after the prefix
    # appends (queued on torch's stream) by the event the pool manager waits on alone.
    hip.gather_host(layout, pool.buffer, [0], [0], [16], [0], 8192)
    waits0 = hip.transfers()["stream_waits"]
    parent = pool.create()
    prefix = [append([parent], [PREFIX], l) for l in range(L)]
    kids = [pool.fork(parent, PREFIX) for _ in range(S)]
    st = pool.stats()
    assert st["shared_blocks"] == L * (PREFIX // B + 1)
    assert st["allocated"] == 1  # a device pool holds its memory from creation
    own = [append(kids, [DIV] * S, l) for l in range(L)]
    hip.check()
    st = pool.stats()
    assert st["cow_copies"] == S * L, st  # the shared partial block, once per child and layer
    assert hip.transfers()["stream_waits"] - waits0 == L  # one ordered COW batch per layer
    # every child reads the shared prefix, then its own rows; the parent is unchanged
    for l in r.choice(L, 3, replace=False):
        pk, pv = read(parent, l)
        assert torch.equal(pk, as_heads(prefix[l][0])) and torch.equal(pv, as_heads(prefix[l][1]))
        for i in r.choice(S, 4, replace=False):
            kk, kv = read(kids[i], l)
            assert torch.equal(kk[:, :PREFIX], pk) and torch.equal(kv[:, :PREFIX], pv)
            assert torch.equal(kk[:, PREFIX:], as_heads(own[l][0][i * DIV:(i + 1) * DIV]))
            assert torch.equal(kv[:, PREFIX:], as_heads(own[l][1][i * DIV:(i + 1) * DIV]))
    # LRU eviction of 25 % of the blocks in use, then compaction under a seeded remap
    for i in r.permutation(S):
        pool.touch(kids[int(i)])
    pool.touch(parent)
    used = N - pool.stats()["free"]
    before = {}
    survivors_probe = [parent] + [kids[int(i)] for i in r.choice(S, 6, replace=False)]
    for s in survivors_probe:
        for l in (0, L // 2, L - 1):
            before[(s, l)] = read(s, l)
    released = pool.evict_lru(used // 4)
    freed = pool.stats()["evicted_blocks"]
    assert freed >= used // 4 and parent not in released
    # first the fewest moves (one batch into the vacant ids), then a full seeded permutation
    for mode, seed in (("fill", 4242), ("permute", 4243)):
        moved = pool.compact(seed=seed, mode=mode)
        assert moved > 0
        st = pool.stats()
        live = N - st["free"]
        for s in survivors_probe:
            if s in released:
                continue
            for l in (0, L // 2, L - 1):
                k, v = read(s, l)
                assert torch.equal(k, before[(s, l)][0]) and torch.equal(v, before[(s, l)][1]), (mode, s, l)
                assert pool.tables([s], l)[0].max() < live
    print(f"  cfg4: {st['cow_copies']} COW copies, {freed} blocks evicted, {moved} moved", flush=True)
    pool.close()


def test_cfg5_sampled(hip):
    """The bench workload's shape and construction at a smaller batch: 48 layers, 4 KV
    heads, GQA 8:1, 8192 positions, tables from the pool manager after seeded alloc/free
    churn (fragmented, as bench.py builds them), one attention launch over every (sequence,
    layer) item of 4 sequences (192 items); 8 sampled items against the oracle."""
    from qubivex_amd import KvLayout, KvPool

    print("cfg5 sampled", flush=True)
    NL, G, D, H, B, CTX, S = 48, 4, 128, 32, 16, 8192, 4
    layout = KvLayout("f16", G, D, B)
    r = np.random.default_rng(505)
    N = int(S * NL * CTX // B * 1.3) + 512
    pool = KvPool(hip, layout, N, NL)
    mem = pool.memory
    dummies, used = [], 0
    while used < int(N * 0.2):  # churn: scatter the free list
        d = pool.create()
        n = int(r.integers(16, 16 * 64))
        pool.plan_append([d], [n], int(r.integers(NL)))
        used += (n + B - 1) // B
        dummies.append(d)
    for i in r.permutation(len(dummies))[: len(dummies) // 2]:
        pool.release(dummies[int(i)])
    seqs = [pool.create() for _ in range(S)]
    gen = torch.Generator(device="cuda").manual_seed(505)
    src = []
    for l in range(NL):
        slots = pool.plan_append(seqs, [CTX] * S, l)
        k = torch.randn((slots.size, G * D), generator=gen, device="cuda")
        v = torch.randn((slots.size, G * D), generator=gen, device="cuda")
        hip.append(layout, mem, N, k, v, t32(slots))
        src.append((k, v))
    hip.check()
    tabs = [pool.tables(seqs, l) for l in range(NL)]
    blocks = np.concatenate([t[0] for t in tabs])
    offs = np.cumsum([0] + [t[0].size for t in tabs[:-1]])
    table_at = np.concatenate([t[1] + o for t, o in zip(tabs, offs)]).astype(np.uint32)
    pos = np.concatenate([t[2] for t in tabs]).astype(np.uint32)
    assert np.array_equal(pos, np.full(S * NL, CTX - 1))
    assert np.mean(np.diff(blocks.astype(np.int64)) != 1) > 0.01  # fragmented tables
    items = S * NL
    q = torch.randn((items, H, D), generator=gen, device="cuda")
    out = torch.empty((items, H, D), device="cuda")
    hip.attention(layout, mem, N, q, t32(blocks), t32(table_at), t32(pos), H, CTX - 1, out)
    hip.check()
    for it in np.sort(r.choice(items, 8, replace=False)):
        l, s = divmod(int(it), S)  # items are layer-major, sequences within a layer
        k, v = src[l]
        kh = k[s * CTX:(s + 1) * CTX].view(CTX, G, D).permute(1, 0, 2).half().float().cpu().numpy()
        vh = v[s * CTX:(s + 1) * CTX].view(CTX, G, D).permute(1, 0, 2).half().float().cpu().numpy()
        want = oracle_attention(kh, vh, q[it].cpu().numpy(), CTX)
        e = attn_errors(out[it].cpu().numpy(), want)
        print(f"  cfg5 item {it} (layer {l}, seq {s}): max_abs={e[0]:.2e} rel_l2={e[1]:.2e}", flush=True)
        assert e[0] <= MAX_ABS and e[1] <= REL_L2, (it, e)
    pool.close()
