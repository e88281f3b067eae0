"""The host-memory entry points (what a Rust DiscreteDevice binds: qvkv_alloc / write /
append / gather / block_copy / decode_attention), concurrent callers on one device, and the
device's counters (usage, transfers)."""
import threading

import numpy as np
import pytest

import oracle
from helpers import MAX_ABS, REL_L2, attn_errors, random_tables, slots_of

pytestmark = pytest.mark.gpu


def test_write_read_round_trip_and_bounds(hip):
    from qubivex_amd import DeviceError

    buf = hip.alloc(4096)
    data = np.arange(1024, dtype=np.uint32).tobytes()
    hip.write(buf, 0, data)
    assert hip.read(buf, 0, 4096) == data
    hip.write(buf, 100, b"\x07" * 8)
    assert hip.read(buf, 100, 8) == b"\x07" * 8
    with pytest.raises(DeviceError):
        hip.write(buf, 4090, b"\x00" * 8)  # past the end: DiscreteDevice::write's error
    u = hip.usage()
    assert u["used"] >= 4096 and u["capacity"] > 200 * 2**30
    buf.close()


@pytest.mark.parametrize("dtype", ["f16", "q8_0"])
def test_host_append_gather_copy_match_the_oracle(hip, dtype):
    from qubivex_amd import KvLayout

    r = np.random.default_rng(31)
    L = KvLayout(dtype, 4, 64, 16)
    N = 24
    buf = hip.alloc(N * L.block_bytes)
    lens = [5, 16, 40]
    blocks, table_at = random_tables(r, lens, 16, N - 6)
    k = r.standard_normal((sum(lens), L.kv_out)).astype(np.float32)
    v = r.standard_normal((sum(lens), L.kv_out)).astype(np.float32)
    slots = np.concatenate([slots_of(blocks, table_at, t, np.arange(n), 16) for t, n in enumerate(lens)])
    hip.append_host(L, buf, k, v, slots)
    sim = oracle.SimPool(N, 4, 64, 16, oracle.F16 if dtype == "f16" else oracle.Q8_0)
    sim.store(k, v, slots)
    out_at = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    gk, gv = hip.gather_host(L, buf, blocks, table_at, lens, out_at, sum(lens))
    for t, n in enumerate(lens):
        wk, wv = sim.gather(blocks, table_at, t, n)
        a = int(out_at[t]) * L.kv_out
        assert np.array_equal(gk[a:a + n * L.kv_out].reshape(4, n, 64), wk)
        assert np.array_equal(gv[a:a + n * L.kv_out].reshape(4, n, 64), wv)
    # copy the first item's block to a free one: the copy reads the same
    free = sorted(set(range(N)) - set(blocks.tolist()))
    hip.block_copy_host(L, buf, [blocks[0]], [free[0]])
    b2 = blocks.copy()
    b2[0] = free[0]
    gk2, _ = hip.gather_host(L, buf, b2, table_at, lens, out_at, sum(lens))
    assert np.array_equal(gk2, gk)
    tr = hip.transfers()
    assert tr["submissions"] > 0 and tr["upload_bytes"] > k.nbytes
    # GPU time of the synchronous calls (TransferStats::timed / gpu_ns)
    hip.append_host(L, buf, k, v, slots)
    t1 = hip.transfers()
    assert t1["timed"] == tr["timed"] + 1 and t1["gpu_ns"] > tr["gpu_ns"]
    assert 0 < hip.timing() < 10**9
    assert hip.max_arena() >= hip.usage()["capacity"] // 2
    buf.close()


def test_host_entry_points_reject_out_of_range_ids(hip):
    from qubivex_amd import KvLayout, ShapeError

    L = KvLayout("f16", 2, 64, 16)
    buf = hip.alloc(4 * L.block_bytes)
    k = np.ones((1, L.kv_out), np.float32)
    with pytest.raises(ShapeError):
        hip.append_host(L, buf, k, k, [4 * 16])
    with pytest.raises(ShapeError):
        hip.block_copy_host(L, buf, [0], [7])
    with pytest.raises(ShapeError):
        hip.gather_host(L, buf, [0], [0], [20], [0], 20)  # one block for 20 positions
    buf.close()


def test_runtime_loop_with_host_authoritative_caches(hip):
    """The reference runtime's decode loop on this library: each pass plans every layer
    with qvkv_pool_plan_attention (attention_plan), copies in the host rows the pool lacks,
    stores the new token and attends (qvkv_decode_attention).  Three sequences, a prompt,
    decode steps, and one cache cleared and refilled (epoch change); every output is
    checked against the oracle's attention over the host cache (f16-narrowed), and the
    counters follow the reference's tests (crates/qubivex-runtime/tests/discrete.rs:692-733):
    the prompt's rows are copied in once per layer and every block returns on drop."""
    from qubivex_amd import KvLayout, KvPool

    r = np.random.default_rng(77)
    G, D, H, L, B = 2, 64, 4, 3, 16
    layout = KvLayout("f16", G, D, B)
    pool = KvPool(hip, layout, 64, L)
    buf = pool.buffer
    seqs = [pool.create() for _ in range(3)]
    prompts = [20, 33, 7]
    host = [[[] for _ in range(L)] for _ in seqs]  # per seq, per layer: list of (k, v) rows
    epochs = [0, 0, 0]
    for i, n in enumerate(prompts):
        for layer in range(L):
            for _ in range(n):
                host[i][layer].append((r.standard_normal(G * D).astype(np.float32),
                                       r.standard_normal(G * D).astype(np.float32)))

    def one_pass():
        pos = [len(host[i][0]) for i in range(len(seqs))]
        for layer in range(L):
            plan = pool.plan_attention(seqs, pos, epochs, layer)
            sync = np.concatenate([np.concatenate(host[int(i)][layer][int(p)])
                                   for i, p in zip(plan["sync_item"], plan["sync_pos"])]
                                  ) if plan["sync_to"].size else np.zeros(0, np.float32)
            kn = r.standard_normal((len(seqs), G * D)).astype(np.float32)
            vn = r.standard_normal((len(seqs), G * D)).astype(np.float32)
            q = r.standard_normal((len(seqs), H, D)).astype(np.float32)
            got = hip.decode_attention(layout, buf, q, H, plan["pos"], plan["blocks"],
                                       plan["table_at"], sync, plan["sync_to"], kn, vn)
            for i in range(len(seqs)):
                host[i][layer].append((kn[i], vn[i]))
                ks = np.stack([k for k, _ in host[i][layer]]).astype(np.float16).astype(np.float32)
                vs = np.stack([v for _, v in host[i][layer]]).astype(np.float16).astype(np.float32)
                for h in range(H):
                    g = h // (H // G)
                    want = oracle.attend(q[i, h], ks[:, g * D:(g + 1) * D], vs[:, g * D:(g + 1) * D],
                                         pos[i])
                    e = attn_errors(got[i, h], want)
                    assert e[0] <= MAX_ABS and e[1] <= REL_L2, (i, layer, h, e)

    one_pass()
    assert pool.stats()["synced_rows"] == sum(prompts) * L
    for _ in range(4):
        one_pass()
    assert pool.stats()["synced_rows"] == sum(prompts) * L  # decode steps copy nothing in
    # sequence 1's cache is cleared and refilled with another prompt: a new epoch
    epochs[1] += 1
    host[1] = [[(r.standard_normal(G * D).astype(np.float32),
                 r.standard_normal(G * D).astype(np.float32)) for _ in range(12)] for _ in range(L)]
    one_pass()
    assert pool.stats()["synced_rows"] == (sum(prompts) + 12) * L
    for s in seqs:
        pool.release(s)
    assert pool.stats()["free"] == pool.stats()["blocks"]
    pool.close()


def test_concurrent_callers_on_one_device(hip):
    """Four threads run decode steps through the host entry point at once (the trait is
    Send + Sync); every result matches its own oracle."""
    from qubivex_amd import KvLayout

    L = KvLayout("f16", 2, 64, 16)
    H = 8
    errors = []

    def worker(seed):
        try:
            r = np.random.default_rng(seed)
            N = 16
            buf = hip.alloc(N * L.block_bytes)
            pos = np.array([int(r.integers(1, 60))], np.uint32)
            blocks, table_at = random_tables(r, [int(pos[0]) + 1], 16, N)
            n = int(pos[0])
            sync = r.standard_normal((n, 2 * L.kv_out)).astype(np.float32)
            sync_to = slots_of(blocks, table_at, 0, np.arange(n), 16)
            kn = r.standard_normal((1, L.kv_out)).astype(np.float32)
            vn = r.standard_normal((1, L.kv_out)).astype(np.float32)
            q = r.standard_normal((1, H, 64)).astype(np.float32)
            for _ in range(5):
                got = hip.decode_attention(L, buf, q, H, pos, blocks, table_at, sync.reshape(-1),
                                           sync_to, kn, vn)
            sim = oracle.SimPool(N, 2, 64, 16, oracle.F16)
            sim.store(sync[:, :L.kv_out], sync[:, L.kv_out:], sync_to)
            sim.store(kn, vn, slots_of(blocks, table_at, 0, [n], 16))
            want = sim.attention(q, H, blocks, table_at, pos)
            e = attn_errors(got, want)
            if not (e[0] <= MAX_ABS and e[1] <= REL_L2):
                errors.append((seed, e))
            buf.close()
        except Exception as ex:  # noqa: BLE001 - reported below
            errors.append((seed, repr(ex)))

    threads = [threading.Thread(target=worker, args=(s,)) for s in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors


def test_split_context_attention_on_concurrent_streams(hip):
    """Four threads, each on its own stream, run attention over one item of 3-5 k
    positions: launches that split the context into chunks, so each needs the partials
    workspace, grown concurrently (the trait is Send + Sync, discrete.rs:433).  Each result
    matches its own oracle.  One thread also passes a block id past its pool on its second
    launch: only its own stream's check reports it."""
    import torch

    from qubivex_amd import KvLayout, ShapeError

    L = KvLayout("f16", 4, 128, 16)
    H = 32
    errors, reported = [], {}

    def worker(seed):
        try:
            r = np.random.default_rng(seed)
            st = torch.cuda.Stream()
            n = int(r.integers(3000, 5000))
            N = n // 16 + 9
            blocks, table_at = random_tables(r, [n], 16, N)
            k = r.standard_normal((n, L.kv_out)).astype(np.float32)
            v = r.standard_normal((n, L.kv_out)).astype(np.float32)
            q = r.standard_normal((1, H, 128)).astype(np.float32)
            slots = slots_of(blocks, table_at, 0, np.arange(n), 16)
            with torch.cuda.stream(st):
                pool = torch.zeros(N * L.block_bytes, dtype=torch.uint8, device="cuda")
                t32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()  # noqa: E731
                dk, dv, dq = (torch.from_numpy(x).cuda() for x in (k, v, q))
                db, dt, dp = t32(blocks), t32(table_at), t32([n - 1])
                bad = t32(np.where(np.arange(blocks.size) == 3, N + 5, blocks))
                out = torch.empty((1, H, 128), device="cuda")
                hip.append(L, pool, N, dk, dv, t32(slots), stream=st)
                sim = oracle.SimPool(N, 4, 128, 16, oracle.F16)
                sim.store(k, v, slots)
                want = sim.attention(q, H, blocks, table_at, np.array([n - 1], np.uint32))
                for it in range(6):
                    out.fill_(float("nan"))
                    tab = bad if (seed == 2 and it == 1) else db
                    hip.attention(L, pool, N, dq, tab, dt, dp, H, n - 1, out, stream=st)
                    try:
                        hip.check(st)
                    except ShapeError:
                        reported[(seed, it)] = True
                        continue
                    e = attn_errors(out.cpu().numpy(), want)
                    if not (e[0] <= MAX_ABS and e[1] <= REL_L2):
                        errors.append((seed, it, e))
        except Exception as ex:  # noqa: BLE001 - reported below
            errors.append((seed, repr(ex)))

    threads = [threading.Thread(target=worker, args=(s,)) for s in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    assert reported == {(2, 1): True}, reported


def test_host_entry_points_reject_null_arrays(hip):
    """A null array with a non-zero count is a ShapeError, not a host crash."""
    import ctypes

    from qubivex_amd import KvLayout, ShapeError, _lib

    L = KvLayout("f16", 2, 64, 16)
    buf = hip.alloc(4 * L.block_bytes)
    lib, lay, dev, pool = _lib.lib, ctypes.byref(L.c), hip.handle, buf.handle
    calls = [
        lambda: lib.qvkv_append(dev, lay, pool, None, None, None, 3),
        lambda: lib.qvkv_gather(dev, lay, pool, None, 4, None, None, None, 2, _lib.F32, 8, None, None),
        lambda: lib.qvkv_block_copy(dev, lay, pool, None, None, 2),
        lambda: lib.qvkv_decode_attention(dev, lay, pool, None, 4, None, 1, None, 1, None, None,
                                          None, 0, None, None, None),
    ]
    for call in calls:
        with pytest.raises(ShapeError):
            _lib.check(call())
    buf.close()


def test_a_dropped_sync_row_is_caught(hip):
    """Positive control for the host-authoritative sync (discrete.rs:951-1009): the same
    call with one sync row left out no longer matches the oracle that has every row."""
    from qubivex_amd import KvLayout

    L = KvLayout("f16", 2, 64, 16)
    H = 8
    r = np.random.default_rng(77)
    N = 8
    n = 50
    pos = np.array([n], np.uint32)
    blocks, table_at = random_tables(r, [n + 1], 16, N)
    sync = r.standard_normal((n, 2 * L.kv_out)).astype(np.float32)
    sync_to = slots_of(blocks, table_at, 0, np.arange(n), 16)
    kn = r.standard_normal((1, L.kv_out)).astype(np.float32)
    vn = r.standard_normal((1, L.kv_out)).astype(np.float32)
    q = (4.0 * r.standard_normal((1, H, 64))).astype(np.float32)  # peaked scores
    sim = oracle.SimPool(N, 2, 64, 16, oracle.F16)
    sim.store(sync[:, :L.kv_out], sync[:, L.kv_out:], sync_to)
    sim.store(kn, vn, slots_of(blocks, table_at, 0, [n], 16))
    want = sim.attention(q, H, blocks, table_at, pos)
    buf = hip.alloc(N * L.block_bytes)
    got = hip.decode_attention(L, buf, q, H, pos, blocks, table_at, sync.reshape(-1), sync_to, kn, vn)
    e = attn_errors(got, want)
    assert e[0] <= MAX_ABS and e[1] <= REL_L2, e
    buf.close()
    buf = hip.alloc(N * L.block_bytes)
    hip.write(buf, 0, bytes(N * L.block_bytes))  # the dropped row reads as zeros
    keep = np.arange(n) != 20
    got = hip.decode_attention(L, buf, q, H, pos, blocks, table_at, sync[keep].reshape(-1),
                               sync_to[keep], kn, vn)
    e = attn_errors(got, want)
    assert not (e[0] <= MAX_ABS and e[1] <= REL_L2), e
    buf.close()


def test_copy_on_write_over_layers_in_one_launch(hip):
    """Children forked from a prefix whose last block is partly filled append on every
    layer through one qvkv_pool_plan_append_layers call: one copy-on-write launch,
    ordered after the prefix appends on torch's stream (one stream wait); every child then
    reads the prefix and its own rows bit for bit, and the parent is unchanged."""
    import torch

    from qubivex_amd import KvLayout, KvPool

    NL, G, D, B = 4, 8, 128, 16
    L = KvLayout("f16", G, D, B)
    N = 256
    pool = KvPool(hip, L, N, NL)
    mem = pool.memory
    gen = torch.Generator(device="cuda").manual_seed(9)
    hip.gather_host(L, pool.buffer, [0], [0], [16], [0], 4096)  # grow the staging first

    def t32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()

    def read(seq, l):
        blocks, table_at, pos = pool.tables([seq], l)
        n = int(pos[0]) + 1
        ok = torch.empty(n * G * D, dtype=torch.float16, device="cuda")
        ov = torch.empty_like(ok)
        hip.gather(L, mem, N, t32(blocks), t32(table_at), t32([n]),
                   torch.zeros(1, dtype=torch.int64, device="cuda"), n, ok, ov, out_dtype="f16")
        hip.check()
        return ok.view(G, n, D), ov.view(G, n, D)

    def heads(x):
        return x.view(-1, G, D).permute(1, 0, 2).half()

    P, DIV, S = 2 * B + 7, 20, 3
    parent = pool.create()
    slots = pool.plan_append_layers([parent], [P], 0, NL)
    pk = torch.randn((slots.size, G * D), generator=gen, device="cuda")
    pv = torch.randn_like(pk)
    hip.append(L, mem, N, pk, pv, t32(slots))  # queued: the copies must wait for it
    kids = [pool.fork(parent, P) for _ in range(S)]
    waits = hip.transfers()["stream_waits"]
    slots = pool.plan_append_layers(kids, [DIV] * S, 0, NL)
    assert hip.transfers()["stream_waits"] == waits + 1
    assert pool.stats()["cow_copies"] == S * NL
    kk = torch.randn((slots.size, G * D), generator=gen, device="cuda")
    kv = torch.randn_like(kk)
    hip.append(L, mem, N, kk, kv, t32(slots))
    for l in range(NL):
        rk, rv = read(parent, l)
        assert torch.equal(rk, heads(pk[l * P:(l + 1) * P])) and torch.equal(rv, heads(pv[l * P:(l + 1) * P]))
        for i, c in enumerate(kids):
            ck, cv = read(c, l)
            own = slice((l * S + i) * DIV, (l * S + i + 1) * DIV)
            assert torch.equal(ck[:, :P], rk) and torch.equal(cv[:, :P], rv), (l, i)
            assert torch.equal(ck[:, P:], heads(kk[own])) and torch.equal(cv[:, P:], heads(kv[own])), (l, i)
    pool.close()


def test_empty_batches_are_no_ops(hip):
    """Every entry point takes an empty batch (no rows, items, segments or pairs) and
    touches nothing: the pool's bytes are unchanged and the error flags stay clear."""
    import ctypes

    import torch

    from qubivex_amd import KvLayout, _lib

    L = KvLayout("f16", 2, 64, 16)
    N = 4
    pool = torch.full((N * L.block_bytes,), 7, dtype=torch.uint8, device="cuda")
    lib, lay, dev = _lib.lib, ctypes.byref(L.c), hip.handle
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = ctypes.c_void_p(pool.data_ptr())
    some = torch.zeros(64, dtype=torch.float32, device="cuda")
    sp = ctypes.c_void_p(some.data_ptr())
    calls = [
        lambda: lib.qvkv_append_async(dev, lay, p, N, sp, sp, sp, 0, st),
        lambda: lib.qvkv_gather_async(dev, lay, p, N, sp, 0, sp, sp, sp, 0, 0, _lib.F32, 0, sp, sp, st),
        lambda: lib.qvkv_attention_async(dev, lay, p, N, sp, sp, 0, sp, sp, 0, 4, 0, sp, st),
        lambda: lib.qvkv_attention_noalloc_async(dev, lay, p, N, sp, sp, 0, sp, sp, 0, 4, 0, sp, st),
        lambda: lib.qvkv_prefill_attention_async(dev, lay, p, N, sp, 0, sp, 0, sp, sp, sp, sp, 0, 4,
                                                 0, 0, sp, st),
        lambda: lib.qvkv_block_copy_async(dev, lay, p, N, sp, sp, 0, st),
    ]
    for call in calls:
        _lib.check(call())
    buf = hip.alloc(N * L.block_bytes)
    hip.write(buf, 0, bytes([7]) * (N * L.block_bytes))
    hip.append_host(L, buf, np.zeros((0, L.kv_out), np.float32), np.zeros((0, L.kv_out), np.float32),
                    np.zeros(0, np.uint32))
    hip.block_copy_host(L, buf, [], [])
    empty = np.zeros(0, np.uint32)
    out = hip.decode_attention(L, buf, np.zeros((0, 4, 64), np.float32), 4, empty, empty, empty,
                               np.zeros(0, np.float32), empty, np.zeros((0, L.kv_out), np.float32),
                               np.zeros((0, L.kv_out), np.float32))
    assert out.shape == (0, 4, 64)
    hip.check()
    assert hip.read(buf, 0, N * L.block_bytes) == bytes([7]) * (N * L.block_bytes)
    assert int((pool != 7).sum()) == 0
    buf.close()


def test_buffers_and_pools_outlive_a_closed_device(hip):
    """qvkv_close before the last buffer and pool are freed (the order a garbage collector
    may pick at teardown): the buffer and the pool are still freed cleanly afterwards (the
    device's struct lives until the last of them)."""
    from qubivex_amd import HipDevice, KvLayout, KvPool

    dev = HipDevice(0)
    buf = dev.alloc(1 << 20)
    dev.write(buf, 0, b"\x01" * 64)
    pool = KvPool(dev, KvLayout("f16", 2, 64, 16), 64, 2)
    dev.close()  # the device first
    buf.close()
    pool.close()
    # the other handle on the same GPU still works
    b2 = hip.alloc(4096)
    hip.write(b2, 0, b"\x02" * 16)
    assert hip.read(b2, 0, 16) == b"\x02" * 16
    b2.close()


def test_graph_replays_of_append_and_attention_match_eager(hip):
    """After one eager step on a stream (which sets up its error flag and workspace), a
    decode step in model order (per layer: append one row per sequence, then attention
    over the layer's items, through the split-by-work path with its merge) is captured into
    a HIP graph on that stream.  Every replay, with eager work and synchronizations between
    replays, gives the eager step's outputs bit for bit; so does the same step through
    qvkv_append_attention_async, captured as well."""
    import torch

    from qubivex_amd import KvLayout, KvPool

    NL, G, D, H, B, S = 3, 8, 128, 32, 16, 8
    L = KvLayout("f16", G, D, B)
    r = np.random.default_rng(5)
    lens = r.integers(100, 3000, size=S)
    N = int(NL * (lens.sum() // B + 2 * S) + 64)
    pool = KvPool(hip, L, N, NL)
    mem = pool.memory
    gen = torch.Generator(device="cuda").manual_seed(5)
    seqs = [pool.create() for _ in range(S)]

    def t32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()

    slots = pool.plan_append_layers(seqs, [int(n) for n in lens], 0, NL)
    k0 = torch.randn((slots.size, G * D), generator=gen, device="cuda")
    hip.append(L, mem, N, k0, torch.randn_like(k0), t32(slots))
    # the step's rows: one new position per sequence and layer (same slots every replay)
    slots = pool.plan_append_layers(seqs, [1] * S, 0, NL)
    d_slots = t32(slots)
    kn = torch.randn((NL * S, G * D), generator=gen, device="cuda")
    vn = torch.randn_like(kn)
    q = torch.randn((NL * S, H * D), generator=gen, device="cuda")
    out = torch.zeros((NL * S, H * D), device="cuda")
    tabs = [pool.tables(seqs, l) for l in range(NL)]
    d_tabs = [(t32(b), t32(ta), t32(p), int(p.max())) for b, ta, p in tabs]
    torch.cuda.synchronize()

    def step():
        for l in range(NL):
            rows = slice(l * S, (l + 1) * S)
            hip.append(L, mem, N, kn[rows], vn[rows], d_slots[rows])
            b, ta, p, mp = d_tabs[l]
            hip.attention(L, mem, N, q[rows], b, ta, p, H, mp, out[rows])

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    s.synchronize()
    hip.check(s)
    ref = out.clone()
    assert torch.isfinite(ref).all()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    torch.cuda.synchronize()
    for rep in range(4):
        out.zero_()
        junk = torch.randn((1 << 20,), generator=gen, device="cuda").sum()  # eager work
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        hip.check(s)
        assert torch.equal(out, ref), rep
        del junk

    # the same step through the fused entry point (one launch per layer), captured too
    def fused_step():
        for l in range(NL):
            rows = slice(l * S, (l + 1) * S)
            b, ta, p, mp = d_tabs[l]
            hip.append_attention(L, mem, N, q[rows], kn[rows], vn[rows], b, ta, p, H, mp,
                                 out[rows])

    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=s):
        fused_step()
    torch.cuda.synchronize()
    for rep in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g2.replay()
        torch.cuda.synchronize()
        hip.check(s)
        assert torch.equal(out, ref), ("fused", rep)
    pool.close()


def test_workspace_growth_on_one_stream_does_not_stall_another(hip):
    """Thread A's attention must grow its stream's workspace, which waits for stream A to
    drain, behind ~0.4 s of queued work.  Meanwhile thread B appends on stream B: its call
    returns while A is still waiting (the wait holds only stream A's lock), and both
    results match the oracle."""
    import time

    import torch

    from qubivex_amd import KvLayout

    L = KvLayout("f16", 4, 128, 16)
    H = 32
    r = np.random.default_rng(77)
    n = 3000
    N = n // 16 + 9
    blocks, table_at = random_tables(r, [n], 16, N)
    k = r.standard_normal((n, L.kv_out)).astype(np.float32)
    v = r.standard_normal((n, L.kv_out)).astype(np.float32)
    q = r.standard_normal((1, H, 128)).astype(np.float32)
    slots = slots_of(blocks, table_at, 0, np.arange(n), 16)
    t32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()  # noqa: E731
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    pool_a = torch.zeros(N * L.block_bytes, dtype=torch.uint8, device="cuda")
    pool_b = torch.zeros(N * L.block_bytes, dtype=torch.uint8, device="cuda")
    dk, dv, dq = (torch.from_numpy(x).cuda() for x in (k, v, q))
    ds, db, dt, dp = t32(slots), t32(blocks), t32(table_at), t32([n - 1])
    out = torch.full((1, H, 128), float("nan"), device="cuda")
    a_mat = torch.randn(8192, 8192, device="cuda")
    torch.cuda.synchronize()
    # each stream's state exists before the timed part (its first use allocates)
    hip.append(L, pool_a, N, dk, dv, ds, stream=sa)
    hip.append(L, pool_b, N, dk[:1], dv[:1], ds[:1], stream=sb)
    hip.check(sa)
    hip.check(sb)
    with torch.cuda.stream(sa):
        for _ in range(40):  # ~0.4 s of work queued on stream A
            a_mat = a_mat @ a_mat * (1.0 / 8192)
    a_done = threading.Event()

    def thread_a():
        hip.attention(L, pool_a, N, dq, db, dt, dp, H, n - 1, out, stream=sa)
        a_done.set()

    ta = threading.Thread(target=thread_a)
    ta.start()
    time.sleep(0.05)
    assert not sa.query(), "stream A drained before the measurement (work too short)"
    t0 = time.perf_counter()
    hip.append(L, pool_b, N, dk, dv, ds, stream=sb)
    dt_b = time.perf_counter() - t0
    a_waiting = not a_done.is_set() and not sa.query()
    ta.join()
    hip.check(sa)
    hip.check(sb)
    print(f"  append on stream B returned in {dt_b * 1e3:.2f} ms; A still waiting: {a_waiting}",
          flush=True)
    assert a_waiting, "stream B's append waited for stream A's workspace growth"
    sim = oracle.SimPool(N, 4, 128, 16, oracle.F16)
    sim.store(k, v, slots)
    want = sim.attention(q, H, blocks, table_at, np.array([n - 1], np.uint32))
    e = attn_errors(out.cpu().numpy(), want)
    assert e[0] <= MAX_ABS and e[1] <= REL_L2, e
    assert torch.equal(pool_a, pool_b)  # B's append stored the same rows


def test_transfer_stats_cover_the_reference_fields(hip):
    """TransferStats (crates/qubivex-compute/src/discrete.rs:376-405) through qvkv_transfers:
    a host-memory call stages its inputs (activations_in), copies its output back
    (activations_out), waits once (fence_waits), and its copies and host time are timed."""
    from qubivex_amd import KvLayout

    r = np.random.default_rng(8)
    L = KvLayout("f16", 2, 64, 16)
    N = 8
    buf = hip.alloc(N * L.block_bytes)
    blocks, table_at = random_tables(r, [40], 16, N)
    k = r.standard_normal((40, L.kv_out)).astype(np.float32)
    v = r.standard_normal((40, L.kv_out)).astype(np.float32)
    slots = slots_of(blocks, table_at, 0, np.arange(40), 16)
    t0 = hip.transfers()
    hip.append_host(L, buf, k, v, slots)
    t1 = hip.transfers()
    assert t1["activations_in"] - t0["activations_in"] >= k.nbytes + v.nbytes + slots.nbytes
    assert t1["fence_waits"] == t0["fence_waits"] + 1
    assert t1["transfer_ns"] > t0["transfer_ns"] and t1["submit_ns"] > t0["submit_ns"]
    out_at = np.zeros(1, np.uint64)
    hip.gather_host(L, buf, blocks, table_at, [40], out_at, 40)
    t2 = hip.transfers()
    assert t2["activations_out"] - t1["activations_out"] == 2 * 40 * L.kv_out * 4
    assert t2["gpu_busy_ns"] == t2["gpu_ns"] and t2["gpu_ns"] > t1["gpu_ns"]
    hip.write(buf, 0, b"\0" * 64)
    t3 = hip.transfers()
    assert t3["activations_in"] == t2["activations_in"]  # a write is not an activation
    assert t3["uploads"] == t2["uploads"] + 1 and t3["fence_waits"] == t2["fence_waits"] + 1
    buf.close()


def test_device_tables_follow_the_pool(hip):
    """qvkv_tables_*: after appends that cross block boundaries, a fork whose child's first
    append copies the shared partial block (copy-on-write: an id changed in place), a
    release and re-create, and a compaction (every id renamed), the device arrays hold
    exactly the pool's tables (qvkv_pool_tables_layers) at item * max_blocks, its pos and
    pos + 1."""
    import torch

    from qubivex_amd import KvLayout, KvPool

    L = KvLayout("f16", 2, 64, 16)
    NL, MB = 3, 40
    pool = KvPool(hip, L, 2000, NL)
    r = np.random.default_rng(4)
    seqs = [pool.create() for _ in range(3)]
    for layer in range(NL):
        pool.plan_append(seqs, [37, 5, 16], layer)
    tables = pool.device_tables(seqs, 0, NL, MB)
    stream = torch.cuda.current_stream()

    def check_mirror():
        mp = tables.sync(stream)
        torch.cuda.synchronize()
        blocks, table_at, pos = pool.tables_layers(seqs, 0, NL)
        n = tables.n_items
        dev = np.frombuffer(hip_read(tables.blocks, tables.n_table), np.uint32)
        dpos = np.frombuffer(hip_read(tables.pos, n), np.uint32)
        dlen = np.frombuffer(hip_read(tables.lens, n), np.uint32)
        dtat = np.frombuffer(hip_read(tables.table_at, n), np.uint32)
        assert dtat.tolist() == [t * MB for t in range(n)]
        assert dpos.tolist() == pos.tolist() and (dlen == pos + 1).all() and mp == int(pos.max())
        ends = list(table_at[1:]) + [blocks.size]
        for t in range(n):
            mine = blocks[table_at[t]:ends[t]]
            assert dev[t * MB:t * MB + mine.size].tolist() == mine.tolist(), t

    def hip_read(ptr, n):
        import ctypes

        rt = ctypes.CDLL("libamdhip64.so.7")  # the HIP runtime already loaded (by soname)
        host = np.zeros(n, np.uint32)
        torch.cuda.synchronize()
        rc = rt.hipMemcpy(ctypes.c_void_p(host.ctypes.data), ctypes.c_void_p(ptr.data_ptr()),
                          ctypes.c_size_t(n * 4), 2)  # hipMemcpyDeviceToHost
        assert rc == 0
        return host.tobytes()

    check_mirror()
    for step in range(40):  # decode steps: one position per layer, blocks appended at edges
        for layer in range(NL):
            pool.plan_append(seqs, [1, 1, 1], layer)
        check_mirror()
    kid = pool.fork(seqs[0], int(pool.length(seqs[0], 0)))
    pool.release(seqs[1])
    seqs2 = [seqs[0], pool.create(), kid]
    for layer in range(NL):
        pool.plan_append(seqs2, [1, 20, 1], layer)  # the kid's append copies the partial block
    tables.close()
    tables = pool.device_tables(seqs2, 0, NL, MB)
    seqs = seqs2
    check_mirror()
    for layer in range(NL):
        pool.plan_append(seqs, [3, 3, 3], layer)
    check_mirror()
    pool.compact(mode="fill")
    check_mirror()
    tables.close()
    pool.close()
