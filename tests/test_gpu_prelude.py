"""The prelude kernel (bias, clip, QK RMSNorm full / per head, RoPE) bit for bit against the
oracle's restatement of the reference's host forward pass, and the prelude + attention
entry point end to end."""
import numpy as np
import pytest

import oracle
from helpers import MAX_ABS, REL_L2, attn_errors, random_tables, slots_of

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def rope_rows(pos, d, base=10000.0):
    """Rope::table rows (crates/qubivex-arch/src/ops.rs:79-92): f64 cos/sin of p*inv_freq."""
    inv = (1.0 / base ** (np.arange(0, d, 2, dtype=np.float64) / d)).astype(np.float32)
    rows = []
    for p in pos:
        a = (np.float32(p) * inv).astype(np.float64)
        rows.append(np.concatenate([np.cos(a), np.sin(a)]).astype(np.float32))
    return np.stack(rows)


CASES = [
    # heads, kv heads, d, norm, clip, bias, scale of inputs
    (32, 8, 128, "full", None, False, 1.0),
    (32, 8, 128, "full", 8.0, True, 20.0),
    (32, 4, 128, "per_head", None, False, 3.0),  # Qwen3-like: declined by the reference device path
    (16, 2, 64, "none", 5.0, True, 10.0),
    (8, 8, 96, "per_head", 2.0, False, 1.0),
    (4, 1, 200, "full", None, True, 1.0),
    # the register kernel (d = 64/128/256 without a full-row norm): partial head batches
    # (12 heads = 8 + 4 at d = 128), pairs across lanes (d = 64), 37 tokens (partial workgroup)
    (64, 8, 256, "per_head", 4.0, True, 2.0),
    (16, 4, 64, "per_head", None, True, 3.0),
    (12, 3, 128, "none", None, True, 1.0),
    (32, 4, 128, "per_head", 6.0, True, 5.0),
    # full-row norms in the register kernel (rows up to 4096 values) and past it (5120)
    (16, 2, 256, "full", None, True, 2.0),
    (64, 8, 64, "full", 3.0, False, 4.0),
    (40, 8, 128, "full", None, True, 1.0),
    # full-row norms whose rows take 2 waves (17-32 values per lane) and k rows of one wave
    (16, 16, 128, "full", 4.0, True, 2.0),
    (24, 2, 64, "full", None, False, 1.0),
]


@pytest.mark.parametrize("fast", [1, 0], ids=["default", "lds_kernel"])
@pytest.mark.parametrize("heads,kvh,d,norm,clip,bias,scale", CASES)
def test_prelude_bit_exact(hip, knobs, heads, kvh, d, norm, clip, bias, scale, fast):
    from qubivex_amd import KvLayout

    # the knob prelude_fast = 0 forces the LDS kernel, the form for every other shape
    knobs("prelude_fast", int(fast))
    print(f"prelude heads={heads} kvh={kvh} d={d} norm={norm} clip={clip} bias={bias} "
          f"fast={fast}", flush=True)
    r = np.random.default_rng(heads * d + kvh)
    L = KvLayout("f16", kvh, d, 16)
    s = 37
    q = (r.standard_normal((s, heads * d)) * scale).astype(np.float32)
    k = (r.standard_normal((s, kvh * d)) * scale).astype(np.float32)
    v = (r.standard_normal((s, kvh * d)) * scale).astype(np.float32)
    rope = rope_rows(r.integers(0, 9000, s), d)
    nq = d if norm == "per_head" else heads * d
    nk = d if norm == "per_head" else kvh * d
    qn = r.uniform(0.5, 1.5, nq).astype(np.float32)
    kn = r.uniform(0.5, 1.5, nk).astype(np.float32)
    qb = r.standard_normal(heads * d).astype(np.float32) if bias else None
    kb = r.standard_normal(kvh * d).astype(np.float32) if bias else None
    vb = r.standard_normal(kvh * d).astype(np.float32) if bias else None
    eps = 1e-6
    code = {"none": 0, "full": 1, "per_head": 2}[norm]
    wq, wk, wv = oracle.prelude(q, k, v, heads, kvh, d, rope, qb, kb, vb, clip, code, qn, kn, eps)
    dq, dk, dv = (torch.from_numpy(x.copy()).cuda() for x in (q, k, v))
    dev = lambda a: None if a is None else torch.from_numpy(a).cuda()  # noqa: E731
    hip.prelude(L, heads, dq, dk, dv, dev(rope), norm=norm, clip=clip, eps=eps,
                q_bias=dev(qb), k_bias=dev(kb), v_bias=dev(vb), q_norm=dev(qn), k_norm=dev(kn))
    hip.check()
    for name, got, want in (("q", dq, wq), ("k", dk, wk), ("v", dv, wv)):
        g = got.cpu().numpy().reshape(-1)
        w = want.reshape(-1)
        bad = np.nonzero(g.view(np.uint32) != w.view(np.uint32))[0]
        assert bad.size == 0, f"{name}: {bad.size} of {g.size} differ, first {bad[:3]}: {g[bad[:3]]} vs {w[bad[:3]]}"


@pytest.mark.parametrize("fast", [1, 0], ids=["default", "lds_kernel"])
@pytest.mark.parametrize("norm,heads,kvh,d", [("per_head", 32, 4, 128), ("full", 16, 2, 128),
                                              ("per_head", 16, 4, 64)])
def test_prelude_norms_follow_the_reduction_tree(hip, knobs, norm, heads, kvh, d, fast):
    """Rows whose sum of squares depends on the order of the additions: each head is
    4096 in one place and +-1 elsewhere, so 2^24 + 1 ties back to 2^24 in a sequential sum
    while reduce.rs's lane tree keeps the ones together (reduce.rs:14-50, pinned by hand in
    test_oracle.py).  The kernel's q and k must equal the oracle's bit for bit, and the
    positive control shows a sequential sum would give a different norm."""
    from qubivex_amd import KvLayout

    knobs("prelude_fast", int(fast))
    r = np.random.default_rng(3)
    L = KvLayout("f16", kvh, d, 16)
    s = 9

    def crafted(n_heads):
        x = np.where(r.random((s, n_heads, d)) < 0.5, -1.0, 1.0).astype(np.float32)
        x[:, :, r.integers(0, d)] = 4096.0
        return x.reshape(s, n_heads * d)

    q, k = crafted(heads), crafted(kvh)
    v = r.standard_normal((s, kvh * d)).astype(np.float32)
    rope = rope_rows(r.integers(0, 9000, s), d)
    nq = d if norm == "per_head" else heads * d
    nk = d if norm == "per_head" else kvh * d
    qn, kn = np.ones(nq, np.float32), np.ones(nk, np.float32)
    code = {"full": 1, "per_head": 2}[norm]
    wq, wk, wv = oracle.prelude(q, k, v, heads, kvh, d, rope, None, None, None, None, code, qn,
                                kn, 1e-6)
    seg = q[0, :nq]
    seq = np.float32(0)
    for x in seg:
        seq = np.float32(np.float32(x * x) + seq)
    assert oracle.reduce_dot(seg, seg) != float(seq)  # the input tells the orders apart
    dq, dk, dv = (torch.from_numpy(x.copy()).cuda() for x in (q, k, v))
    hip.prelude(L, heads, dq, dk, dv, torch.from_numpy(rope).cuda(), norm=norm, eps=1e-6,
                q_norm=torch.from_numpy(qn).cuda(), k_norm=torch.from_numpy(kn).cuda())
    hip.check()
    for name, got, want in (("q", dq, wq), ("k", dk, wk)):
        g = got.cpu().numpy().reshape(-1)
        assert np.array_equal(g.view(np.uint32), want.reshape(-1).view(np.uint32)), name


def test_prelude_attention_end_to_end(hip):
    """qvkv_prelude_attention: projection outputs in; post-prelude rows stored after the
    sync rows; attention of the post-prelude q; k_new / v_new back bit for bit."""
    from qubivex_amd import KvLayout

    r = np.random.default_rng(5)
    heads, kvh, d, B = 16, 4, 128, 16
    L = KvLayout("f16", kvh, d, B)
    N = 64
    buf = hip.alloc(N * L.block_bytes)
    pos = np.array([0, 37, 100], np.uint32)
    s = pos.size
    blocks, table_at = random_tables(r, (pos + 1).tolist(), B, N)
    sync_rows, sync_to = [], []
    for t, p in enumerate(pos):
        for j in range(int(p)):
            sync_rows.append(r.standard_normal(2 * L.kv_out).astype(np.float32))
            sync_to.append(int(slots_of(blocks, table_at, t, [j], B)[0]))
    sync = np.concatenate(sync_rows)
    sync_to = np.array(sync_to, np.uint32)
    q = (r.standard_normal((s, heads * d)) * 4).astype(np.float32)
    k = (r.standard_normal((s, kvh * d)) * 4).astype(np.float32)
    v = (r.standard_normal((s, kvh * d)) * 4).astype(np.float32)
    rope = rope_rows(pos, d)
    qn = r.uniform(0.5, 1.5, heads * d).astype(np.float32)
    kn = r.uniform(0.5, 1.5, kvh * d).astype(np.float32)
    out, k_new, v_new = hip.prelude_attention(L, buf, heads, q, k, v, rope, pos, blocks, table_at,
                                              sync, sync_to, norm="full", clip=6.0, eps=1e-5,
                                              q_norm=qn, k_norm=kn)
    wq, wk, wv = oracle.prelude(q, k, v, heads, kvh, d, rope, clip=6.0, norm=1, q_norm=qn,
                                k_norm=kn, eps=1e-5)
    assert np.array_equal(k_new.view(np.uint32), wk.reshape(s, -1).view(np.uint32))
    assert np.array_equal(v_new.view(np.uint32), wv.reshape(s, -1).view(np.uint32))
    sim = oracle.SimPool(N, kvh, d, B, oracle.F16)
    sr = sync.reshape(-1, 2 * L.kv_out)
    sim.store(sr[:, :L.kv_out], sr[:, L.kv_out:], sync_to)
    new_slots = np.array([slots_of(blocks, table_at, t, [int(p)], B)[0] for t, p in enumerate(pos)],
                         np.uint32)
    sim.store(wk.reshape(s, -1), wv.reshape(s, -1), new_slots)
    want = sim.attention(wq.reshape(s, heads, d), heads, blocks, table_at, pos)
    e = attn_errors(out, want)
    assert e[0] <= MAX_ABS and e[1] <= REL_L2, e
    buf.close()
