"""Paged prefill attention (qvkv_prefill_attention_async) against the oracle: every token
of a segment attends causally over positions 0..pos0+j of its sequence, as the
reference's host prefill runs math::attend per (token, head) after storing the segment
(crates/qubivex-arch/src/lib.rs:1296-1320).  The oracle expands each segment into one
decode item per token."""
import numpy as np
import pytest

import oracle
from helpers import F16, MAX_ABS, Q8_0, REL_L2, attn_errors, decode_pool, normal, rng, slots_of
from test_gpu_kernels import cf32, cu32, fill_items, layout, new_pool

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def expand(table_at, lens, n_tok, q_at):
    """Per-token (table_at, pos, q row) of the segments; sequence i ends at lens[i]."""
    ta, pos, rows = [], [], []
    for i, (n, m) in enumerate(zip(lens, n_tok)):
        for j in range(m):
            ta.append(table_at[i])
            pos.append(n - m + j)
            rows.append(q_at[i] + j)
    return (np.array(ta, np.uint32), np.array(pos, np.uint32), np.array(rows, np.int64))


PREFILL_CASES = [
    # dtype, H, G, D, [(sequence length after the segment, tokens in the segment)]
    (F16, 32, 8, 128, [(512, 512), (300, 37), (17, 1), (1000, 130)]),  # 4 heads per KV head
    (F16, 32, 4, 128, [(64, 64), (2000, 33), (16, 16)]),  # 8 per KV head
    (F16, 8, 8, 128, [(100, 100), (45, 9)]),  # 1 per KV head: 8 tokens per wave
    (F16, 16, 1, 128, [(90, 90)]),  # 16 per KV head
    (F16, 8, 2, 64, [(200, 200), (77, 5)]),
    (F16, 12, 4, 128, [(50, 50), (81, 3)]),  # 3 per KV head: waves straddle tokens
    (F16, 4, 2, 256, [(300, 40)]),
    (F16, 4, 4, 96, [(60, 60), (129, 7)]),  # generic kernel
    (Q8_0, 32, 8, 128, [(256, 256), (700, 45)]),
    (Q8_0, 32, 4, 128, [(300, 300), (33, 2)]),
    (Q8_0, 8, 2, 64, [(130, 66)]),
    (Q8_0, 4, 2, 256, [(90, 20)]),
    (Q8_0, 6, 3, 160, [(70, 12)]),  # generic kernel
    # query groups that are not powers of two
    (F16, 12, 2, 128, [(200, 37), (45, 45)]),
    (F16, 24, 2, 128, [(130, 20)]),
    (Q8_0, 12, 4, 128, [(150, 40), (17, 17)]),
    (Q8_0, 10, 2, 128, [(99, 33)]),
    (F16, 12, 4, 64, [(80, 30)]),
]


@pytest.mark.parametrize("dtype,H,G,D,segs", PREFILL_CASES)
def test_prefill_within_tolerance(hip, dtype, H, G, D, segs):
    print(f"prefill {dtype} H={H} G={G} D={D} segs={segs}", flush=True)
    r = rng(900 + H * G + D + len(segs))
    L = layout(dtype, G, D)
    lens = [n for n, _ in segs]
    n_tok = np.array([m for _, m in segs], np.uint32)
    N = sum((n + 15) // 16 for n in lens) + 5
    pool = new_pool(L, N, fill=9)
    blocks, table_at, sim = fill_items(hip, L, pool, N, lens, r,
                                       outliers=0.01 if dtype == Q8_0 else 0)
    # segments' q rows in reverse order: q_at is an indirection, not the segment index
    T = int(n_tok.sum())
    q_at = np.zeros(len(segs), np.uint32)
    at = 0
    for i in reversed(range(len(segs))):
        q_at[i] = at
        at += int(n_tok[i])
    pos0 = (np.array(lens, np.uint32) - n_tok).astype(np.uint32)
    q = normal(r, (T, H, D))
    out = torch.full((T * H * D,), float("nan"), dtype=torch.float32, device="cuda")
    max_pos = int(max(lens)) - 1
    hip.prefill_attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32(pos0),
                          cu32(q_at), cu32(n_tok), H, max_pos, int(n_tok.max()), out)
    hip.check()
    got = out.cpu().numpy().reshape(T, H, D)
    ta, pos, rows = expand(table_at, lens, n_tok, q_at)
    want = sim.attention(q[rows], H, blocks, ta, pos)
    max_abs, rel = attn_errors(got[rows], want)
    print(f"  max_abs={max_abs:.2e} rel_l2={rel:.2e}", flush=True)
    assert np.isfinite(got).all()
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)


@pytest.mark.parametrize("dtype,D", [(F16, 128), (F16, 64), (Q8_0, 128)])
def test_prefill_reads_no_table_entry_past_a_segment(hip, dtype, D):
    """Each segment's table is followed by an id far past the pool.  The segments end 1-16
    positions into a last tile whose count is a multiple of 3 (so the streaming loop's
    three-tile steps end just before it, and the tile's second half starts past the
    context): the kernel must resolve no table entry for that half, so no error is
    latched, and the results match the oracle."""
    print(f"prefill table tail {dtype} D={D}", flush=True)
    r = rng(77 + D)
    H = G = 8   # one query row per token: a 64-token segment is one workgroup
    L = layout(dtype, G, D)
    segs = [(261, 64), (360, 64), (944, 64), (1025, 40)]
    lens = [n for n, _ in segs]
    n_tok = np.array([m for _, m in segs], np.uint32)
    N = sum((n + 15) // 16 for n in lens) + 5
    pool = new_pool(L, N, fill=9)
    blocks, table_at, sim = fill_items(hip, L, pool, N, lens, r)
    padded, padded_at = [], []
    for i, n in enumerate(lens):
        padded_at.append(len(padded))
        padded.extend(blocks[table_at[i]:table_at[i] + (n + 15) // 16])
        padded.append(0xFFFFFFFF)
    padded = np.array(padded, np.uint32)
    padded_at = np.array(padded_at, np.uint32)
    T = int(n_tok.sum())
    q_at = np.concatenate([[0], np.cumsum(n_tok)[:-1]]).astype(np.uint32)
    pos0 = (np.array(lens, np.uint32) - n_tok).astype(np.uint32)
    q = normal(r, (T, H, D))
    out = torch.full((T * H * D,), float("nan"), dtype=torch.float32, device="cuda")
    hip.prefill_attention(L, pool, N, cf32(q), cu32(padded), cu32(padded_at), cu32(pos0),
                          cu32(q_at), cu32(n_tok), H, int(max(lens)) - 1, int(n_tok.max()), out)
    hip.check()
    got = out.cpu().numpy().reshape(T, H, D)
    ta, pos, rows = expand(table_at, lens, n_tok, q_at)
    want = sim.attention(q[rows], H, blocks, ta, pos)
    max_abs, rel = attn_errors(got[rows], want)
    print(f"  max_abs={max_abs:.2e} rel_l2={rel:.2e}", flush=True)
    assert max_abs <= MAX_ABS and rel <= REL_L2, (max_abs, rel)


@pytest.mark.parametrize("exact_p", [True, False])
def test_prefill_equals_decode_kernel_per_token(hip, exact_p, knobs):
    """The prefill kernel and the decode kernel (one item per token) agree to float
    rounding on the same pool: the same tiles, scores and softmax, another order (with
    the prefill's P as high part + residual); with P as one f16 (the default prefill)
    to its rounding, 2^-11 relative per probability."""
    if exact_p:
        knobs("prefill_exact_p", 1)
    r = rng(31)
    L = layout(F16, 8, 128)
    H = 32
    lens, n_tok = [700], np.array([200], np.uint32)
    N = 50
    pool = new_pool(L, N)
    blocks, table_at, _ = fill_items(hip, L, pool, N, lens, r)
    q = normal(r, (200, H, 128))
    pos0 = np.array([500], np.uint32)
    a = torch.zeros(200 * H * 128, dtype=torch.float32, device="cuda")
    b = torch.zeros_like(a)
    hip.prefill_attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32(pos0),
                          cu32(np.zeros(1, np.uint32)), cu32(n_tok), H, 699, 200, a)
    pos = np.arange(500, 700, dtype=np.uint32)
    hip.attention(L, pool, N, cf32(q), cu32(blocks), cu32(np.zeros(200, np.uint32)), cu32(pos),
                  H, 699, b)
    hip.check()
    d = (a - b).abs().max().item()
    assert d < (1e-5 if exact_p else 2e-4), d


@pytest.mark.parametrize("dtype,D", [(F16, 64), (F16, 128), (Q8_0, 128), (Q8_0, 64)])
def test_prefill_rejects_out_of_range_segments(hip, dtype, D):
    """A segment past max_pos, past max_tok, past q_rows or past its table is a ShapeError
    and the kernel touches nothing; a block id past the pool is a ShapeError too (every
    prefill form: register-staged f16, DMA f16, q8_0 MFMA, decode-tile)."""
    from qubivex_amd import ShapeError

    r = rng(32)
    L = layout(dtype, 2, D)
    N = 8
    pool = new_pool(L, N)
    blocks, table_at, _ = fill_items(hip, L, pool, N, [40], r)
    q = cf32(normal(r, (10, 4, D)))
    out = torch.zeros(10 * 4 * D, dtype=torch.float32, device="cuda")
    args = dict(blocks=cu32(blocks), table_at=cu32(table_at))
    bad = [
        (np.array([35], np.uint32), np.array([0], np.uint32), np.array([10], np.uint32), 40, 10),  # max_pos
        (np.array([30], np.uint32), np.array([0], np.uint32), np.array([10], np.uint32), 39, 5),  # max_tok
        (np.array([30], np.uint32), np.array([5], np.uint32), np.array([10], np.uint32), 39, 10),  # q rows
        (np.array([40], np.uint32), np.array([0], np.uint32), np.array([10], np.uint32), 60, 10),  # table
    ]
    for pos0, q_at, n_tok, max_pos, max_tok in bad:
        hip.prefill_attention(L, pool, N, q, args["blocks"], args["table_at"], cu32(pos0),
                              cu32(q_at), cu32(n_tok), 4, max_pos, max_tok, out)
        with pytest.raises(ShapeError):
            hip.check()
    assert float(out.abs().sum()) == 0.0
    # a block id past the pool in the segment's table
    bad_blocks = blocks.copy()
    bad_blocks[1] = N + 5
    hip.prefill_attention(L, pool, N, q, cu32(bad_blocks), args["table_at"], cu32([30]),
                          cu32([0]), cu32([10]), 4, 39, 10, out)
    with pytest.raises(ShapeError):
        hip.check()
    hip.check()  # cleared


def test_host_entry_routes_a_prefill_chunk_through_segments(hip):
    """qvkv_decode_attention with a prompt chunk of one sequence, a decode token of
    another and a second chunk: the runs become prefill segments; the results are those
    of attending each token on its own."""
    from qubivex_amd import KvLayout

    r = rng(33)
    L = KvLayout(F16, 4, 128, 16)
    H = 16
    N = 60
    buf = hip.alloc(N * L.block_bytes)
    # sequence 0: positions 0..39 new; sequence 1: 1 new token at 300; sequence 2: 100..119
    lens = [40, 301, 120]
    blocks = r.permutation(N).astype(np.uint32)[:sum((n + 15) // 16 for n in lens)]
    need = [(n + 15) // 16 for n in lens]
    table_at_seq = np.concatenate([[0], np.cumsum(need)[:-1]]).astype(np.uint32)
    toks = [(0, p) for p in range(40)] + [(1, 300)] + [(2, p) for p in range(100, 120)]
    s = len(toks)
    pos = np.array([p for _, p in toks], np.uint32)
    table_at = np.array([table_at_seq[i] for i, _ in toks], np.uint32)
    # host rows of everything before the new tokens: synced now
    sync_rows, sync_to = [], []
    for i, first_new in ((1, 300), (2, 100)):
        for j in range(first_new):
            sync_rows.append(normal(r, (2 * L.kv_out,)))
            sync_to.append(int(slots_of(blocks, table_at_seq, i, [j], 16)[0]))
    sync = np.concatenate(sync_rows)
    sync_to = np.array(sync_to, np.uint32)
    k_new = normal(r, (s, L.kv_out))
    v_new = normal(r, (s, L.kv_out))
    q = normal(r, (s, H, 128))
    got = hip.decode_attention(L, buf, q, H, pos, blocks, table_at, sync, sync_to, k_new, v_new)
    sim = oracle.SimPool(N, 4, 128, 16, oracle.F16)
    sr = sync.reshape(-1, 2 * L.kv_out)
    sim.store(sr[:, :L.kv_out], sr[:, L.kv_out:], sync_to)
    new_slots = np.array([slots_of(blocks, table_at_seq, i, [p], 16)[0] for i, p in toks], np.uint32)
    sim.store(k_new, v_new, new_slots)
    want = sim.attention(q, H, blocks, table_at, pos)
    max_abs, rel = attn_errors(got, want)
    print(f"  max_abs={max_abs:.2e} rel_l2={rel:.2e}", flush=True)
    assert max_abs <= MAX_ABS and rel <= REL_L2
    buf.close()


def _f64_attention(k16, v16, q, g_of, npos):
    """Exact attention of one query over positions 0..npos-1 (float64)."""
    s = k16[:npos, g_of] @ q.astype(np.float64) / np.sqrt(q.size)
    p = np.exp(s - s.max())
    return p @ v16[:npos, g_of] / p.sum()


@pytest.mark.parametrize("kind", ["prefill", "prefill_exact_p", "decode"])
def test_f16_paths_track_float64_closely(hip, kind, knobs):
    """With f16 K/V the products q.k and p.v are exact in the MFMAs when q and p are
    carried as f16 high part + residual (decode, and the prefill with
    knob prefill_exact_p = 1): those paths sit within ~1e-6 of float64.  Pins the split: a
    high part and residual taken from two different roundings of the same product (a
    contraction into v_fma_mix for one of them) leaves one-ulp errors that show up here
    as ~1e-5.  The default prefill carries P as one f16 (relative error 2^-11 per
    probability, normalised by the sum of the rounded values): about 2e-5 here, held
    under 2e-4, ten times inside the reference tolerance of 2e-3."""
    if kind == "prefill_exact_p":
        knobs("prefill_exact_p", 1)
    r = rng(77)
    G, D, H = 4, 128, 32
    L = layout(F16, G, D)
    n, nt = 1500, 40
    N = (n + 15) // 16 + 2
    pool = new_pool(L, N)
    blocks, table_at, _ = fill_items(hip, L, pool, N, [n], r)
    raw = pool.cpu().numpy()
    dec = decode_pool(raw, L, N)
    k16 = np.zeros((n, G, D)); v16 = np.zeros((n, G, D))
    for p in range(n):
        b, o = blocks[p // 16], p % 16
        k16[p] = dec["k"][b, :, o].view(np.float16).astype(np.float64)
        v16[p] = dec["v"][b, :, o].view(np.float16).astype(np.float64)
    q = normal(r, (nt, H, D))
    out = torch.zeros(nt * H * D, dtype=torch.float32, device="cuda")
    if kind.startswith("prefill"):
        hip.prefill_attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at),
                              cu32([n - nt]), cu32([0]), cu32([nt]), H, n - 1, nt, out)
    else:
        pos = np.arange(n - nt, n, dtype=np.uint32)
        hip.attention(L, pool, N, cf32(q), cu32(blocks), cu32(np.zeros(nt, np.uint32)),
                      cu32(pos), H, n - 1, out)
    hip.check()
    got = out.cpu().numpy().reshape(nt, H, D)
    worst = 0.0
    for j in range(nt):
        for h in range(H):
            worst = max(worst, np.abs(got[j, h] - _f64_attention(k16, v16, q[j, h], h // (H // G),
                                                                 n - nt + j + 1)).max())
    print(f"  {kind}: max |got - f64| = {worst:.2e}", flush=True)
    assert worst < (2e-4 if kind == "prefill" else 1e-5), worst


@pytest.mark.parametrize("kind", ["prefill", "decode"])
def test_q8_0_paths_track_float64_closely(hip, kind):
    """q8_0 values are exact in both kernels: decode converts int8 to f16 and applies the
    scales in f32; the MFMA prefill keeps keys as int8 and splits each dequantised value
    into an f16 high part and its exact residual (products then carry ~2^-22 relative
    error).  Against float64 attention over the dequantised pool both stay within 1e-6
    of the largest value magnitude (outliers x8 included: |v| up to ~40; measured about
    1e-5 absolute, against the reference tolerance of 2e-3)."""
    r = rng(78)
    G, D, H = 8, 128, 32
    L = layout(Q8_0, G, D)
    n, nt = 1200, 40
    N = (n + 15) // 16 + 2
    pool = new_pool(L, N)
    blocks, table_at, _ = fill_items(hip, L, pool, N, [n], r, outliers=0.01)
    dec = decode_pool(pool.cpu().numpy(), L, N)
    kd = np.zeros((n, G, D)); vd = np.zeros((n, G, D))
    grp = np.arange(D) // 32
    for p in range(n):
        b, o = blocks[p // 16], p % 16
        ks = dec["ks"][b, :, o].view(np.float16).astype(np.float64)
        vs = dec["vs"][b, :, o].view(np.float16).astype(np.float64)
        kd[p] = dec["k"][b, :, o].astype(np.float64) * ks[:, grp]
        vd[p] = dec["v"][b, :, o].astype(np.float64) * vs[:, grp]
    q = normal(r, (nt, H, D))
    out = torch.zeros(nt * H * D, dtype=torch.float32, device="cuda")
    if kind.startswith("prefill"):
        hip.prefill_attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at),
                              cu32([n - nt]), cu32([0]), cu32([nt]), H, n - 1, nt, out)
    else:
        pos = np.arange(n - nt, n, dtype=np.uint32)
        hip.attention(L, pool, N, cf32(q), cu32(blocks), cu32(np.zeros(nt, np.uint32)),
                      cu32(pos), H, n - 1, out)
    hip.check()
    got = out.cpu().numpy().reshape(nt, H, D)
    worst = 0.0
    for j in range(nt):
        for h in range(H):
            worst = max(worst, np.abs(got[j, h] - _f64_attention(kd, vd, q[j, h], h // (H // G),
                                                                 n - nt + j + 1)).max())
    bound = 1e-6 * np.abs(vd).max()
    print(f"  {kind}: max |got - f64| = {worst:.2e} (bound {bound:.2e})", flush=True)
    assert worst < bound, (worst, bound)


def test_q8_0_prefill_reports_value_scales_past_its_range(hip):
    """The MFMA prefill holds dequantised values in f16: a value scale above 512 is
    reported as UnsupportedError instead of producing infinities; the same pool through
    decode attention (f32 scales) is fine."""
    from qubivex_amd import UnsupportedError
    r = rng(79)
    G, D, H = 2, 128, 8
    L = layout(Q8_0, G, D)
    n = 64
    N = n // 16 + 2
    pool = new_pool(L, N)
    blocks, table_at, _ = fill_items(hip, L, pool, N, [n], r)
    k = normal(r, (1, L.kv_out)) * 1e5  # amax / 127 > 512
    v = normal(r, (1, L.kv_out)) * 1e5
    hip.append(L, pool, N, cf32(k), cf32(v), cu32(slots_of(blocks, table_at, 0, [n - 1], 16)))
    hip.check()
    q = normal(r, (1, H, D))
    out = torch.zeros(H * D, dtype=torch.float32, device="cuda")
    hip.prefill_attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32([n - 1]),
                          cu32([0]), cu32([1]), H, n - 1, 1, out)
    with pytest.raises(UnsupportedError, match="scale above 512"):
        hip.check()
    hip.attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32([n - 1]), H, n - 1, out)
    hip.check()
    assert np.isfinite(out.cpu().numpy()).all()


@pytest.mark.parametrize("dtype,H,G,D", [(F16, 32, 8, 128), (Q8_0, 32, 8, 128), (F16, 16, 4, 64),
                                         (Q8_0, 8, 2, 64), (F16, 8, 2, 256)])
def test_prefill_with_a_dominant_position(hip, dtype, H, G, D):
    """The prefill kernels' row max over a tile, with one key scaled x40 in each row group
    and in later tiles (see test_attention_with_a_dominant_position)."""
    from test_gpu_kernels import dominant_items
    print(f"prefill dominant {dtype} H={H} G={G} D={D}", flush=True)
    r = rng(600 + D + G)
    L = layout(dtype, G, D)
    lens = [40, 40, 40, 40, 200]
    big = [3, 7, 11, 15, 100]
    N, pool, blocks, table_at, sim, _ = dominant_items(hip, L, H, r, lens, big)
    nt = 20  # the last 20 tokens of each item as one segment
    q = normal(r, (len(lens) * nt, H, D))
    pos0 = np.array(lens, np.uint32) - nt
    q_at = np.arange(len(lens), dtype=np.uint32) * nt
    out = torch.full((q.size,), float("nan"), dtype=torch.float32, device="cuda")
    hip.prefill_attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32(pos0),
                          cu32(q_at), cu32([nt] * len(lens)), H, max(lens) - 1, nt, out)
    hip.check()
    got = out.cpu().numpy().reshape(len(lens), nt, H, D)
    worst = (0.0, 0.0)
    for t, n in enumerate(lens):
        pos = np.arange(n - nt, n, dtype=np.uint32)
        want = sim.attention(q[t * nt:(t + 1) * nt], H, blocks,
                             np.full(nt, table_at[t], np.uint32), pos)
        assert np.isfinite(got[t]).all(), t
        max_abs, rel = attn_errors(got[t], want)
        worst = (max(worst[0], max_abs), max(worst[1], rel))
    print(f"  max_abs={worst[0]:.2e} rel_l2={worst[1]:.2e}", flush=True)
    assert worst[0] <= MAX_ABS and worst[1] <= REL_L2, worst


def test_host_entry_recomputes_a_q8_0_chunk_past_the_f16_range(hip):
    """qvkv_decode_attention with a q8_0 prompt chunk whose values pass the f16 range
    (scales above 512): the MFMA prefill reports the range, and the synchronous entry point
    recomputes the chunk with the f32-scale form, so the call succeeds and matches the
    oracle (relative tolerance: the values are ~1e5)."""
    from qubivex_amd import KvLayout

    r = rng(34)
    L = KvLayout(Q8_0, 2, 128, 16)
    H = 8
    n = 40
    N = 8
    buf = hip.alloc(N * L.block_bytes)
    blocks = r.permutation(N).astype(np.uint32)[:(n + 15) // 16]
    pos = np.arange(n, dtype=np.uint32)
    table_at = np.zeros(n, np.uint32)
    k_new = normal(r, (n, L.kv_out))
    v_new = normal(r, (n, L.kv_out)) * 1e5
    q = normal(r, (n, H, 128))
    got = hip.decode_attention(L, buf, q, H, pos, blocks, table_at,
                               np.zeros(0, np.float32), np.zeros(0, np.uint32), k_new, v_new)
    sim = oracle.SimPool(N, 2, 128, 16, oracle.Q8_0)
    slots = slots_of(blocks, np.zeros(1, np.uint32), 0, pos, 16)
    sim.store(k_new, v_new, slots)
    want = sim.attention(q, H, blocks, table_at, pos)
    assert np.isfinite(got).all()
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    print(f"  rel_l2={rel:.2e}", flush=True)
    assert rel <= REL_L2
    buf.close()
