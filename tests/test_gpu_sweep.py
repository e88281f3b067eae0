"""Seeded random shapes through every attention entry point, against the oracle.

The fixed-shape tests pin each kernel form on chosen cases; this sweep draws the shape
parameters together (pool dtype, head dim including the generic kernel's, KV heads, query
heads per KV head up to two head chunks, block size, ragged context lengths with block-edge
values, launch form), so that combinations no list names still meet the oracle:
  * decode attention within max-abs 2e-3 / relative L2 1e-3 of the oracle's `attend`
    (the reference's sequential f32 order, crates/qubivex-compute/src/math.rs:120-155),
    on a pool whose unwritten slots hold random bytes;
  * prefill attention of a random segment per sequence within the same bounds, each token
    checked as the decode item the reference's host prefill runs
    (crates/qubivex-arch/src/lib.rs:1296-1320);
  * the fused append + attention bit for bit against the append followed by attention;
  * append (f16 narrowing, q8_0 quantisation), gather and block copy bit for bit against
    the oracle's f16 / q8_0 encoders (crates/qubivex-compute/src/math.rs:13-60,
    formats.rs:21-99) and its simulated pool, rows scaled over 1e-6..300 with specials.
Each case prints its parameters first, so a failure names them."""
import numpy as np
import pytest

import oracle
from helpers import F16, MAX_ABS, Q8_0, REL_L2, attn_errors, decode_pool, normal, rng
from test_gpu_kernels import EDGE_F32, cf32, cu32, cu64, fill_items, is_nan16, layout, new_pool
from test_gpu_prefill import expand

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

# launch forms of a decode attention launch, chosen by the library's tuning variables
FORMS = {
    "default": {},
    "unsplit": {"attn_full": "1"},                                   # one workgroup per unit
    "work": {"attn_full": "1000000000", "attn_stream": "1"},    # split by work
    "chunks": {"attn_full": "1000000000", "attn_stream": "0"},  # context chunks
}


def draw(seed):
    r = np.random.default_rng(seed)
    dtype = F16 if r.random() < 0.5 else Q8_0
    dims = [64, 128, 128, 256, 96, 200, 512, 8] if dtype == F16 else [64, 128, 128, 256, 96, 160, 512]
    D = int(r.choice(dims))
    G = int(r.integers(1, 9))
    GS = int(r.choice([1, 2, 3, 4, 5, 6, 8, 12, 16]))
    B = int(r.choice([16, 16, 32, 48, 256]))
    n = int(r.integers(1, 20))
    # the oracle runs a few GFLOP/s: longest context bounded to ~3 GFLOP of decode work
    top = int(np.clip(3e9 / (4 * G * GS * D * n), 2 * B + 2, 2600))
    lens = [int(x) for x in r.integers(1, top + 1, n)]
    for i in range(n):  # block edges
        if r.random() < 0.3:
            lens[i] = max(1, int(r.choice([1, B - 1, B, B + 1, 2 * B])))
    form = str(r.choice(list(FORMS)))
    return dtype, D, G, G * GS, B, lens, form


SEEDS = list(range(7000, 7100))


@pytest.mark.parametrize("seed", SEEDS)
def test_random_shapes_match_the_oracle(hip, seed, knobs):
    dtype, D, G, H, B, lens, form = draw(seed)
    print(f"sweep seed={seed} {dtype} D={D} G={G} H={H} B={B} form={form} lens={lens}", flush=True)
    for k, v in FORMS[form].items():
        knobs(k, int(v))
    r = rng(seed)
    L = layout(dtype, G, D, B)
    N = sum((x + B - 1) // B for x in lens) + 3
    pool = new_pool(L, N, fill=seed)
    blocks, table_at, sim = fill_items(hip, L, pool, N, lens, r,
                                       outliers=0.01 if dtype == Q8_0 else 0)

    # decode attention at each sequence's last position
    q = normal(r, (len(lens), H, D))
    pos = np.array(lens, np.uint32) - 1
    out = torch.full((len(lens) * H * D,), float("nan"), dtype=torch.float32, device="cuda")
    hip.attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32(pos), H, int(pos.max()), out)
    hip.check()
    got = out.cpu().numpy().reshape(len(lens), H, D)
    want = sim.attention(q, H, blocks, table_at, pos)
    max_abs, rel = attn_errors(got, want)
    print(f"  attention max_abs={max_abs:.2e} rel_l2={rel:.2e}", flush=True)
    assert np.isfinite(got).all()
    assert max_abs <= MAX_ABS and rel <= REL_L2, ("attention", max_abs, rel)

    # prefill: a random trailing segment of each sequence (at most 96 tokens, fewer where
    # the oracle's work would pass ~4 GFLOP), q rows in a shuffled order
    cap = int(np.clip(4e9 / (4 * H * D * sum(lens)), 1, 96))
    n_tok = np.array([int(r.integers(1, min(x, cap) + 1)) for x in lens], np.uint32)
    T = int(n_tok.sum())
    order = r.permutation(len(lens))
    q_at = np.zeros(len(lens), np.uint32)
    at = 0
    for i in order:
        q_at[i] = at
        at += int(n_tok[i])
    pos0 = (np.array(lens, np.uint32) - n_tok).astype(np.uint32)
    qp = normal(r, (T, H, D))
    outp = torch.full((T * H * D,), float("nan"), dtype=torch.float32, device="cuda")
    hip.prefill_attention(L, pool, N, cf32(qp), cu32(blocks), cu32(table_at), cu32(pos0),
                          cu32(q_at), cu32(n_tok), H, int(max(lens)) - 1, int(n_tok.max()), outp)
    hip.check()
    gotp = outp.cpu().numpy().reshape(T, H, D)
    ta, pp, rows = expand(table_at, lens, n_tok, q_at)
    wantp = sim.attention(qp[rows], H, blocks, ta, pp)
    max_abs, rel = attn_errors(gotp[rows], wantp)
    print(f"  prefill max_abs={max_abs:.2e} rel_l2={rel:.2e}", flush=True)
    assert np.isfinite(gotp).all()
    assert max_abs <= MAX_ABS and rel <= REL_L2, ("prefill", max_abs, rel)


@pytest.mark.parametrize("seed", SEEDS[::2])
def test_random_shapes_fused_append_attention(hip, seed, knobs):
    from test_gpu_append_attention import run_case

    dtype, D, G, H, B, lens, form = draw(seed)
    run_case(hip, "f16" if dtype == F16 else "q8_0", G, H, D, B, lens, FORMS[form], knobs)


@pytest.mark.parametrize("seed", SEEDS[1::2])
def test_random_shapes_store_gather_and_copy_bytes(hip, seed):
    dtype, D, G, H, B, lens, _ = draw(seed)
    print(f"bytes seed={seed} {dtype} D={D} G={G} B={B} items={len(lens)}", flush=True)
    r = rng(seed + 1)
    L = layout(dtype, G, D, B)

    # append at random slots of a zeroed pool: every stored code against the oracle's encoder
    N = int(r.integers(2, 40))
    n = int(r.integers(1, min(N * B, 300) + 1))
    slots = r.choice(N * B, n, replace=False).astype(np.uint32)
    k = normal(r, (n, G * D), 0.01) * np.float32(r.choice([1e-6, 1e-3, 1.0, 300.0], (n, 1)))
    v = normal(r, (n, G * D), 0.01)
    m = min(EDGE_F32.size, G * D)
    k[0, :m] = EDGE_F32[:m]
    v[-1, :m] = -EDGE_F32[:m]
    pool = new_pool(L, N)
    hip.append(L, pool, N, cf32(k), cf32(v), cu32(slots))
    hip.check()
    dec = decode_pool(pool.cpu().numpy(), L, N)
    b, o = slots // B, slots % B
    for name, x in (("k", k), ("v", v)):
        got = dec[name][b, :, o]                       # [n][G][D]
        if dtype == F16:
            want = oracle.f16_bits(x).reshape(n, G, D)
            ok = (got == want) | (is_nan16(got) & is_nan16(want))
            assert ok.all(), (name, np.argwhere(~ok)[:4])
        else:
            want = oracle.q8_0_quantize(x).reshape(n, G, D // 32, 34)
            wscale = want[..., 0].astype(np.uint16) | (want[..., 1].astype(np.uint16) << 8)
            gscale = dec[name + "s"][b, :, o]
            assert ((gscale == wscale) | (is_nan16(gscale) & is_nan16(wscale))).all(), name + " scales"
            assert (got == want[..., 2:].view(np.int8).reshape(n, G, D)).all(), name + " values"
    written = np.zeros(N * B, bool)
    written[slots] = True
    keys = dec["k"].transpose(0, 2, 1, 3).reshape(N * B, G, D)
    assert not keys[~written].any()

    # gather of ragged items through shuffled tables, f32 (and f16 for f16 pools)
    glens = [min(x, 700) for x in lens]
    N = sum((x + B - 1) // B for x in glens) + 3
    pool = new_pool(L, N, fill=seed)
    blocks, table_at, sim = fill_items(hip, L, pool, N, glens, r)
    out_at = np.concatenate([[0], np.cumsum(glens)[:-1]]).astype(np.uint64)
    total = int(sum(glens))
    for od in (["f32", "f16"] if dtype == F16 else ["f32"]):
        tdt = torch.float32 if od == "f32" else torch.float16
        ok_ = torch.full((total * L.kv_out,), 7, dtype=tdt, device="cuda")
        ov_ = torch.full_like(ok_, 7)
        hip.gather(L, pool, N, cu32(blocks), cu32(table_at), cu32(glens), cu64(out_at),
                   max(glens), ok_, ov_, out_dtype=od)
        hip.check()
        gk, gv = ok_.cpu().numpy(), ov_.cpu().numpy()
        for t, x in enumerate(glens):
            wk, wv = sim.gather(blocks, table_at, t, x)
            a, e = int(out_at[t]) * L.kv_out, (int(out_at[t]) + x) * L.kv_out
            if od == "f32":
                assert np.array_equal(gk[a:e].view(np.uint32), wk.reshape(-1).view(np.uint32)), t
                assert np.array_equal(gv[a:e].view(np.uint32), wv.reshape(-1).view(np.uint32)), t
            else:
                assert np.array_equal(gk[a:e].view(np.uint16), oracle.f16_bits(wk)), t
                assert np.array_equal(gv[a:e].view(np.uint16), oracle.f16_bits(wv)), t

    # block copy between disjoint random block sets
    before = pool.cpu().numpy().reshape(N, -1).copy()
    ids = r.permutation(N)
    c = int(r.integers(1, N // 2 + 1))
    src, dst = ids[:c].astype(np.uint32), ids[c:2 * c].astype(np.uint32)
    hip.block_copy(L, pool, N, cu32(src), cu32(dst))
    hip.check()
    want = before.copy()
    want[dst] = before[src]
    assert np.array_equal(pool.cpu().numpy().reshape(N, -1), want)
