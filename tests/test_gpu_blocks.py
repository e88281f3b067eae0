"""Block sizes other than 16: every kernel addresses positions as block * B + offset with a
16-position tile inside one block, so B = 32, 48 (not a power of two), 256 (the reference's
KV_BLOCK, crates/qubivex-compute/src/discrete.rs:247-329) and 4096 (the largest) must give
the same results.  Append and gather bit for bit; decode and prefill attention within the
reference tolerance."""
import numpy as np
import pytest

from helpers import F16, MAX_ABS, Q8_0, REL_L2, attn_errors, normal, rng
from test_gpu_kernels import cf32, cu32, cu64, fill_items, layout, new_pool

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.mark.parametrize("B", [32, 48, 256, 4096])
@pytest.mark.parametrize("dtype", [F16, Q8_0])
def test_block_sizes(hip, dtype, B):
    print(f"blocks {dtype} B={B}", flush=True)
    r = rng(1000 + B + (dtype == Q8_0))
    G, D, H = 4, 128, 16
    L = layout(dtype, G, D, B)
    lens = [1, 15, 17, 33, B - 1, B, B + 1, 3 * B + 5, 700]
    N = sum((n + B - 1) // B for n in lens) + 3
    pool = new_pool(L, N, fill=7)
    blocks, table_at, sim = fill_items(hip, L, pool, N, lens, r,
                                       outliers=0.01 if dtype == Q8_0 else 0)

    # gather: the logical values of every position, bit for bit
    total = int(sum(lens))
    out_at = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    ok = torch.empty(total * L.kv_out, dtype=torch.float32, device="cuda")
    ov = torch.empty_like(ok)
    hip.gather(L, pool, N, cu32(blocks), cu32(table_at), cu32(np.array(lens, np.uint32)),
               cu64(out_at), max(lens), ok, ov, "f32")
    hip.check()
    gk, gv = ok.cpu().numpy(), ov.cpu().numpy()
    for t, n in enumerate(lens):
        wk, wv = sim.gather(blocks, table_at, t, n)
        o = int(out_at[t]) * L.kv_out
        assert np.array_equal(gk[o:o + G * n * D].view(np.uint32),
                              wk.reshape(-1).view(np.uint32)), (t, n)
        assert np.array_equal(gv[o:o + G * n * D].view(np.uint32),
                              wv.reshape(-1).view(np.uint32)), (t, n)

    # decode attention of the last position of every item
    q = normal(r, (len(lens), H, D))
    pos = np.array(lens, np.uint32) - 1
    out = torch.zeros(len(lens) * H * D, dtype=torch.float32, device="cuda")
    hip.attention(L, pool, N, cf32(q), cu32(blocks), cu32(table_at), cu32(pos), H,
                  int(pos.max()), out)
    hip.check()
    e = attn_errors(out.cpu().numpy().reshape(len(lens), H, D),
                    sim.attention(q, H, blocks, table_at, pos))
    print(f"  decode max_abs={e[0]:.2e} rel_l2={e[1]:.2e}", flush=True)
    assert e[0] <= MAX_ABS and e[1] <= REL_L2, e

    # prefill: the last min(n, 40) tokens of every item as one segment each
    n_tok = np.minimum(np.array(lens), 40).astype(np.uint32)
    pos0 = (np.array(lens) - n_tok).astype(np.uint32)
    q_at = np.concatenate([[0], np.cumsum(n_tok)[:-1]]).astype(np.uint32)
    T = int(n_tok.sum())
    qp = normal(r, (T, H, D))
    outp = torch.zeros(T * H * D, dtype=torch.float32, device="cuda")
    hip.prefill_attention(L, pool, N, cf32(qp), cu32(blocks), cu32(table_at), cu32(pos0),
                          cu32(q_at), cu32(n_tok), H, int(max(lens)) - 1, int(n_tok.max()), outp)
    hip.check()
    ta = np.repeat(table_at, n_tok).astype(np.uint32)
    pt = np.concatenate([np.arange(p, p + m) for p, m in zip(pos0, n_tok)]).astype(np.uint32)
    e = attn_errors(outp.cpu().numpy().reshape(T, H, D), sim.attention(qp, H, blocks, ta, pt))
    print(f"  prefill max_abs={e[0]:.2e} rel_l2={e[1]:.2e}", flush=True)
    assert e[0] <= MAX_ABS and e[1] <= REL_L2, e
