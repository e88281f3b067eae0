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
  * the fused append + attention bit for bit against the append followed by attention.
Each case prints its parameters first, so a failure names them."""
import numpy as np
import pytest

from helpers import F16, MAX_ABS, Q8_0, REL_L2, attn_errors, normal, rng
from test_gpu_kernels import cf32, cu32, fill_items, layout, new_pool
from test_gpu_prefill import expand

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

# launch forms of a decode attention launch, chosen by the library's tuning variables
FORMS = {
    "default": {},
    "unsplit": {"QVKV_ATTN_FULL": "1"},                                   # one workgroup per unit
    "work": {"QVKV_ATTN_FULL": "1000000000", "QVKV_ATTN_STREAM": "1"},    # split by work
    "chunks": {"QVKV_ATTN_FULL": "1000000000", "QVKV_ATTN_STREAM": "0"},  # context chunks
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
def test_random_shapes_match_the_oracle(hip, seed, monkeypatch):
    dtype, D, G, H, B, lens, form = draw(seed)
    print(f"sweep seed={seed} {dtype} D={D} G={G} H={H} B={B} form={form} lens={lens}", flush=True)
    for k, v in FORMS[form].items():
        monkeypatch.setenv(k, v)
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
def test_random_shapes_fused_append_attention(hip, seed, monkeypatch):
    from test_gpu_append_attention import run_case

    dtype, D, G, H, B, lens, form = draw(seed)
    run_case(hip, "f16" if dtype == F16 else "q8_0", G, H, D, B, lens, FORMS[form], monkeypatch)
