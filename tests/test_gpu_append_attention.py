"""qvkv_append_attention_async: the step's new key and value rows stored at each item's
position, then attention over 0..pos -- the reference's DeviceMoeAttention submission after
its sync rows (crates/qubivex-compute/src/discrete.rs:257-307).  It must give, bit for bit,
the outputs and the pool bytes of qvkv_append_async at the same slots followed by
qvkv_attention_async (whose parity with the oracle the attention tests pin), on every
launch form (one workgroup per unit, the split by work, the context-chunk split), for f16
and q8_0 pools (q8_0: the new rows quantised as the append stores them), and on the unfused
paths (head dims without an MFMA kernel, or the knob fused_q8 = 0)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

CASES = [
    # dtype, kv heads, query heads, d, block, sequence lengths before the step, env
    ("f16", 8, 32, 128, 16, [300, 17, 4096, 1000, 64, 1], {}),             # split by work
    ("f16", 4, 32, 128, 16, [2049, 15, 16, 31, 33] * 26, {}),              # one per unit
    ("f16", 8, 32, 128, 16, [3000, 700, 129], {"attn_stream": "0"}),  # context chunks
    ("f16", 2, 32, 128, 32, [95, 96, 97, 500], {}),                        # 2 head chunks
    ("f16", 8, 16, 64, 16, [200, 47, 1], {}),
    ("f16", 4, 8, 256, 256, [600, 255, 256], {}),
    ("q8_0", 8, 32, 128, 16, [300, 1000, 31], {}),                         # split by work
    ("q8_0", 4, 32, 128, 16, [2049, 15, 16, 31, 33] * 26, {}),             # one per unit
    ("q8_0", 8, 32, 128, 16, [1000, 17, 64, 4095] * 32, {}),               # one per unit, packed
    ("q8_0", 8, 32, 128, 16, [3000, 700, 129], {"attn_stream": "0"}),  # context chunks
    ("q8_0", 2, 32, 128, 32, [95, 96, 97, 500], {}),                       # 2 head chunks
    ("q8_0", 8, 16, 64, 16, [200, 47, 1], {}),
    ("q8_0", 4, 8, 256, 256, [600, 255, 256], {}),
    ("q8_0", 8, 32, 128, 16, [300, 31], {"fused_q8": "0"}),           # unfused
    ("f16", 4, 8, 96, 16, [100, 33], {}),                                  # unfused (generic)
]


@pytest.mark.parametrize("dtype,G,H,D,B,lens,env", CASES)
def test_append_attention_equals_append_then_attention(hip, dtype, G, H, D, B, lens, env,
                                                       knobs):
    run_case(hip, dtype, G, H, D, B, lens, env, knobs)


@pytest.mark.parametrize("dtype,lens,env", [
    ("f16", [300, 17, 64], {}), ("f16", [2049, 15] * 130, {}),
    ("q8_0", [300, 17, 64], {}), ("q8_0", [2049, 15] * 130, {}),
])
def test_append_attention_with_special_values_in_the_new_rows(hip, dtype, lens, env, knobs):
    """NaN, infinities, values past the f16 range, f32 subnormals and an all-zero q8_0 group
    in the step's new rows: the fused launch narrows or quantises them exactly as the append
    (compared bit for bit, NaN outputs included)."""
    run_case(hip, dtype, 8, 32, 128, 16, lens, env, knobs, special=True)


def run_case(hip, dtype, G, H, D, B, lens, env, knobs, special=False):
    from qubivex_amd import KvLayout, KvPool

    print(f"append+attention {dtype} G={G} H={H} D={D} B={B} items={len(lens)} env={env} "
          f"special={special}", flush=True)
    for k, v in env.items():
        knobs(k, int(v))
    L = KvLayout(dtype, G, D, B)
    S = len(lens)
    N = sum(n // B + 2 for n in lens) + 8
    pool = KvPool(hip, L, N, 1)
    mem = pool.memory
    gen = torch.Generator(device="cuda").manual_seed(len(lens) * 7 + D)
    seqs = [pool.create() for _ in range(S)]

    def t32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()

    slots = pool.plan_append(seqs, lens, 0)
    k0 = torch.randn((slots.size, G * D), generator=gen, device="cuda")
    hip.append(L, mem, N, k0, torch.randn_like(k0), t32(slots))
    new = pool.plan_append(seqs, [1] * S, 0)  # the step's positions
    blocks, table_at, pos = pool.tables(seqs, 0)
    assert (pos == np.array(lens)).all()
    kn = torch.randn((S, G * D), generator=gen, device="cuda")
    vn = torch.randn_like(kn)
    if special:
        odd = torch.tensor([float("nan"), float("inf"), -float("inf"), 1e30, -1e30, 1e-40,
                            65520.0, 6e-8], device="cuda")
        kn[0, :8] = odd
        vn[0, 8:16] = odd
        kn[1 % S, 32:64] = 0.0  # an all-zero q8_0 group
        vn[1 % S, 32:64] = 0.0
        kn[2 % S, D:D + 8] = odd.flip(0)
    q = torch.randn((S, H * D), generator=gen, device="cuda")
    d_b, d_t, d_p = t32(blocks), t32(table_at), t32(pos)
    torch.cuda.synchronize()
    size = N * L.block_bytes
    before = hip.read(pool.buffer, 0, size)

    out_a = torch.full((S, H * D), float("nan"), device="cuda")
    hip.append(L, mem, N, kn, vn, t32(new))
    hip.attention(L, mem, N, q, d_b, d_t, d_p, H, int(pos.max()), out_a)
    torch.cuda.synchronize()
    hip.check()
    pool_a = hip.read(pool.buffer, 0, size)

    hip.write(pool.buffer, 0, before)
    out_b = torch.full((S, H * D), float("nan"), device="cuda")
    hip.append_attention(L, mem, N, q, kn, vn, d_b, d_t, d_p, H, int(pos.max()), out_b)
    torch.cuda.synchronize()
    hip.check()
    pool_b = hip.read(pool.buffer, 0, size)

    if not special:
        assert torch.isfinite(out_a).all()
    assert torch.equal(out_a.view(torch.int32), out_b.view(torch.int32))
    assert pool_a == pool_b
    assert pool_a != before  # the rows were stored
    pool.close()


def test_append_attention_reports_range_errors(hip):
    """A position past max_pos or past its table is a ShapeError, as for attention."""
    from qubivex_amd import KvLayout, KvPool, ShapeError

    for dtype in ("f16", "q8_0"):
        L = KvLayout(dtype, 2, 128, 16)
        pool = KvPool(hip, L, 16, 1)
        seq = pool.create()
        pool.plan_append([seq], [40], 0)
        blocks, table_at, pos = pool.tables([seq], 0)

        def t32(a):
            return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()

        kn = torch.zeros((1, 256), device="cuda")
        q = torch.zeros((1, 8 * 128), device="cuda")
        out = torch.zeros_like(q)
        hip.append_attention(L, pool.memory, 16, q, kn, kn, t32(blocks), t32(table_at),
                             t32(pos), 8, int(pos[0]) - 1, out)  # pos past max_pos
        with pytest.raises(ShapeError):
            hip.check()
        hip.append_attention(L, pool.memory, 16, q, kn, kn, t32(blocks[:2]), t32(table_at),
                             t32(pos), 8, int(pos[0]), out)  # table too short
        with pytest.raises(ShapeError):
            hip.check()
        hip.check()
        pool.close()
