"""The allocation-free attention entry point (qvkv_attention_noalloc_async) through the C
ABI: its output equals qvkv_attention_async's bit for bit on two calls in a row (the
second smaller, so the scratch array holds the first call's partials when it starts), on
launches that split the context (the ones that use the scratch).  A launch needing more
scratch than the array holds is refused before it starts."""
import ctypes

import numpy as np
import pytest

from helpers import random_tables, slots_of

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def t32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()


def _call(fn, hip, L, pool, N, q, blocks, table_at, pos, H, max_pos, out):
    from qubivex_amd import _lib

    st = torch.cuda.current_stream().cuda_stream
    return fn(hip.handle, ctypes.byref(L.c), ctypes.c_void_p(pool.data_ptr()), N,
              ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(blocks.data_ptr()), blocks.numel(),
              ctypes.c_void_p(table_at.data_ptr()), ctypes.c_void_p(pos.data_ptr()), pos.numel(),
              H, max_pos, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(st))


@pytest.mark.parametrize("dtype", ["f16", "q8_0"])
def test_noalloc_attention_equals_the_allocating_form(hip, dtype):
    from qubivex_amd import KvLayout, _lib

    print(f"noalloc {dtype}", flush=True)
    L = KvLayout(dtype, 4, 128, 16)
    H = 32
    r = np.random.default_rng(7)
    lens = [4100, 2500, 9000]
    N = sum((n + 15) // 16 for n in lens) + 8
    blocks, table_at = random_tables(r, lens, 16, N)
    pool = torch.zeros(N * L.block_bytes, dtype=torch.uint8, device="cuda")
    slots = np.concatenate([slots_of(blocks, table_at, t, np.arange(n), 16)
                            for t, n in enumerate(lens)])
    k = torch.randn((slots.size, L.kv_out), device="cuda")
    v = torch.randn((slots.size, L.kv_out), device="cuda")
    hip.append(L, pool, N, k, v, t32(slots))
    hip.check()
    for n_items in (3, 1):  # the second call smaller than the first
        q = torch.randn((n_items, H, 128), device="cuda")
        pos = np.array([n - 1 for n in lens[:n_items]], np.uint32)
        max_pos = int(pos.max())
        want = torch.full((n_items, H, 128), float("nan"), device="cuda")
        got = torch.full_like(want, float("nan"))
        _lib.check(_call(_lib.lib.qvkv_attention_async, hip, L, pool, N, q, t32(blocks),
                         t32(table_at), t32(pos), H, max_pos, want))
        hip.check()
        tb, tt, tp = t32(blocks), t32(table_at), t32(pos)
        torch.cuda.synchronize()
        u0, (f0, _) = hip.usage(), torch.cuda.mem_get_info()
        _lib.check(_call(_lib.lib.qvkv_attention_noalloc_async, hip, L, pool, N, q, tb, tt, tp,
                         H, max_pos, got))
        hip.check()
        u1, (f1, _) = hip.usage(), torch.cuda.mem_get_info()
        # nothing allocated: the library's own accounting and the device's free memory
        assert (u1["used"], u1["peak"]) == (u0["used"], u0["peak"]), (u0, u1)
        assert f1 == f0, (f0, f1)
        assert torch.isfinite(want).all()
        assert torch.equal(got, want), (n_items, float((got - want).abs().max()))


def test_noalloc_attention_refuses_a_launch_past_its_scratch(hip, knobs):
    from qubivex_amd import KvLayout, ShapeError, _lib

    # a tiny launch over a long context split by work over as many workgroups as it has
    # 4-tile shares (8192 here): 2 partial slots x 8 heads x 258 floats per workgroup need
    # more than the scratch array holds
    knobs("attn_stream_wg", 100000)
    L = KvLayout("f16", 1, 256, 16)
    q = torch.zeros((8, 8, 256), device="cuda")
    out = torch.zeros_like(q)
    ids = t32(np.zeros(8, np.uint32))
    pool = torch.zeros(L.block_bytes, dtype=torch.uint8, device="cuda")
    rc = _call(_lib.lib.qvkv_attention_noalloc_async, hip, L, pool, 1, q, ids, ids, ids, 8,
               65535, out)
    assert rc == _lib.E_SHAPE
    code, msg = _lib.last_error()
    assert "scratch" in msg
    with pytest.raises(ShapeError):
        _lib.check(rc)
    assert float(out.abs().sum()) == 0.0  # nothing ran
