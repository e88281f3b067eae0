"""Benchmark of the paged KV-cache hot path on one MI355X.

Headline workload ("cfg5"): Qwen3-30B-A3B-like KV, 48 layers,
4 KV heads, head_dim 128, 32 query heads (GQA 8:1), f16 storage, block 16, 128 sequences
at 8192 context (~103 GB of KV resident).  Block tables come from the library's pool
manager after seeded alloc/free churn (fragmented).  The pool is filled by bulk
prefill-appends of 512 tokens x all sequences x all layers per call (the timed append leg).

One step = one decode step: one append per sequence on every layer (its newest position)
plus paged decode attention of every query head over the whole context on every layer,
as one attention launch over all (sequence, layer) items; value = tokens/s = sequences /
step time.  Inputs are resident in HBM before the timed region.  Also timed:
  * the same step in model order: per layer, append + attention over that layer's 128
    items (layer l+1's query depends on layer l), 48 launch pairs per step;
  * block-table gather, batched block copy, paged prefill attention and the prelude;
  * the CPU baseline: the oracle's restatement of the reference CPU path (gather +
    `attend`, OpenMP over heads) on 8 seeded (sequence, layer) items of the timed step,
    whose K/V are read back raw from the pool; the same leg checks the timed GPU output
    of those items against it (the line carries "validated").
Then the other BASELINE.json configurations run in the same process (keys under
"configs"): cfg1 (latency loop), cfg2 (batched decode, ragged contexts), cfg3 (q8_0),
cfg4 (prefix sharing: copy-on-write, LRU eviction, compaction on 64 KiB blocks).
`--config cfgN` makes another configuration the headline; `--only` skips the others.
"""
import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_F16_TFLOPS = 2500.0  # dense f16 MFMA, MI355X

CONFIGS = {
    # layers, kv heads, head dim, q heads, sequences, context (int or (lo, hi)), dtype, outliers
    "cfg5": dict(layers=48, kv_heads=4, head_dim=128, q_heads=32, seqs=128, ctx=8192,
                 dtype="f16", outliers=0.0, qk_norm="per_head",
                 name="cfg5 (Qwen3-30B-A3B-like KV, 128 seqs x 8192)"),
    "cfg2": dict(layers=32, kv_heads=8, head_dim=128, q_heads=32, seqs=32, ctx=(256, 4096),
                 dtype="f16", outliers=0.0,
                 name="cfg2 (Llama-3-8B-like KV, 32 seqs x U[256,4096])"),
    "cfg3": dict(layers=32, kv_heads=8, head_dim=128, q_heads=32, seqs=64, ctx=2048,
                 dtype="q8_0", outliers=0.01,
                 name="cfg3 (q8_0 KV, 64 seqs x 2048, 1% x8 outliers)"),
    "cfg4": dict(layers=32, kv_heads=8, head_dim=128, seqs=64, prefix=2047, divergent=256,
                 dtype="f16", name="cfg4 (prefix sharing: 64 seqs on a 2047-token prefix)"),
    "cfg1": dict(layers=16, kv_heads=8, head_dim=64, q_heads=32, prefill=512, decode=128,
                 dtype="f16", name="cfg1 (small Llama-like KV, one sequence)"),
}
DECODE_CONFIGS = ("cfg5", "cfg2", "cfg3")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="cfg5", choices=DECODE_CONFIGS)
    ap.add_argument("--only", action="store_true", help="skip the other configurations")
    ap.add_argument("--configs", default="cfg2,cfg3,cfg4,cfg1",
                    help="the other configurations to run after the headline (comma list)")
    ap.add_argument("--seqs", type=int, default=None, help="override the config's sequences")
    ap.add_argument("--ctx", type=int, default=None, help="override the config's context")
    ap.add_argument("--layers", type=int, default=None, help="override the config's layers")
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--legs", default="append,decode,layers,gather,copy,prefill,prelude")
    ap.add_argument("--tune", action="append", default=[], metavar="KNOB=VALUE",
                    help="set a launch-shape knob (qvkv_tune) before running, for A/B runs")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Timer:
    """HIP events on the stream the timed kernels run on (torch's current stream, which
    the bindings launch on)."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream

    def __call__(self, fn, reps):
        ev = self.torch.cuda.Event
        e0, e1 = ev(enable_timing=True), ev(enable_timing=True)
        e0.record(self.stream)
        for _ in range(reps):
            fn()
        e1.record(self.stream)
        self.torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps


def cu32(torch, a):
    import numpy as np

    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()


# --------------------------------------------------------------------------------------
# decode configurations (cfg5 headline, cfg2, cfg3)
# --------------------------------------------------------------------------------------

def run_decode(name, args, dev, legs, steps, warmup, cpu):
    import numpy as np
    import torch

    from qubivex_amd import KvLayout, KvPool

    cfg = dict(CONFIGS[name])
    if name == args.config:
        for key in ("seqs", "ctx", "layers"):
            if getattr(args, key) is not None:
                cfg[key] = getattr(args, key)
    S, NL = cfg["seqs"], cfg["layers"]
    G, D, H, B = cfg["kv_heads"], cfg["head_dim"], cfg["q_heads"], 16
    dtype = cfg["dtype"]
    L = KvLayout(dtype, G, D, B)
    kv_out = G * D
    bytes_per_value = 2 if dtype == "f16" else 34 / 32
    r = np.random.default_rng(args.seed)
    if isinstance(cfg["ctx"], tuple):
        ctx = r.integers(cfg["ctx"][0], cfg["ctx"][1] + 1, S)
    else:
        ctx = np.full(S, cfg["ctx"])
    real_blocks = int(sum((int(c) + B - 1) // B for c in ctx)) * NL
    n_blocks = int(real_blocks * 1.25) + 1024
    log(f"[bench] {cfg['name']}; pool {n_blocks} blocks x {L.block_bytes} B = "
        f"{n_blocks * L.block_bytes / 1e9:.1f} GB")
    pool = KvPool(dev, L, n_blocks, NL)
    mem = pool.memory
    stream = torch.cuda.current_stream()
    timer = Timer(torch, stream)
    c32 = lambda a: cu32(torch, a)  # noqa: E731

    # ---- seeded churn: scatter the free list before the real sequences allocate
    dummies, used = [], 0
    while used < int(n_blocks * 0.2):
        s = pool.create()
        n = int(r.integers(16, 16 * 64))
        pool.plan_append([s], [n], int(r.integers(NL)))
        used += (n + B - 1) // B
        dummies.append(s)
    order = r.permutation(len(dummies))
    for i in order[: len(order) // 2]:
        pool.release(dummies[i])
    keep = [dummies[i] for i in order[len(order) // 2:]]
    seqs = [pool.create() for _ in range(S)]

    # ---- fill: bulk prefill-append of up to CHUNK tokens per sequence, all layers per call
    CHUNK = 512
    gen = torch.Generator(device="cuda").manual_seed(args.seed)
    append_ms, append_bytes = [], []
    fill_to = ctx - 1  # the decode step writes each sequence's position ctx-1
    filled = np.zeros(S, np.int64)
    t0 = time.time()
    while (filled < fill_to).any():
        counts = np.minimum(CHUNK, fill_to - filled).astype(np.uint32)
        slots = np.concatenate([pool.plan_append(seqs, counts, l) for l in range(NL)])
        n_rows = slots.size
        sl = c32(slots)
        k = torch.randn((n_rows, kv_out), generator=gen, device="cuda", dtype=torch.float32)
        v = torch.randn((n_rows, kv_out), generator=gen, device="cuda", dtype=torch.float32)
        if cfg["outliers"]:
            for x in (k, v):
                x[torch.rand(x.shape, generator=gen, device="cuda") < cfg["outliers"]] *= 8.0
        if not filled.any():
            # untimed warm-up: the process's first launch of the kernel pays its code load
            # (about 3x the launch's time); the same rows written again are the same bytes
            dev.append(L, mem, n_blocks, k, v, sl)
        ms = timer(lambda: dev.append(L, mem, n_blocks, k, v, sl), 1)
        dev.check()
        if (counts == CHUNK).all():
            append_ms.append(ms)
            append_bytes.append(n_rows * kv_out * (4 * 2 + 2 * bytes_per_value) + n_rows * 4)
        filled += counts
        del k, v, sl
    for s in keep:
        pool.release(s)
    log(f"[bench] filled {int(fill_to.sum())} positions x {NL} layers ({time.time() - t0:.1f}s)")

    # ---- the decode step's inputs: one new token per (sequence, layer) at position ctx-1
    slots = np.concatenate([pool.plan_append(seqs, [1] * S, l) for l in range(NL)])
    tabs = [pool.tables(seqs, l) for l in range(NL)]
    blocks = np.concatenate([t[0] for t in tabs])
    offs = np.cumsum([0] + [t[0].size for t in tabs[:-1]])
    table_at = np.concatenate([t[1] + o for t, o in zip(tabs, offs)]).astype(np.uint32)
    pos = np.concatenate([t[2] for t in tabs]).astype(np.uint32)
    items = pos.size
    assert items == S * NL and np.array_equal(pos, np.tile(ctx - 1, NL))
    frag = float(np.mean(np.diff(blocks.astype(np.int64)) != 1))
    d_slots, d_blocks, d_tat, d_pos = c32(slots), c32(blocks), c32(table_at), c32(pos)
    kn = torch.randn((items, kv_out), generator=gen, device="cuda")
    vn = torch.randn((items, kv_out), generator=gen, device="cuda")
    q = torch.randn((items, H, D), generator=gen, device="cuda")
    out = torch.empty((items, H, D), device="cuda")
    max_pos = int(pos.max())
    positions = float(np.sum(pos.astype(np.float64) + 1))
    kv_bytes_step = positions * kv_out * 2 * bytes_per_value
    attn_bytes = kv_bytes_step + q.numel() * 4 * 2 + blocks.size * 4 + items * 8
    flops = 4.0 * H * D * positions
    # MFMA work the decode kernel issues: per 16-position tile of one (item, KV head, chunk
    # of <= 8 query heads) 2*d/16 v_mfma_f32_16x16x16_f16 (QK^T and PV), 4096 FMA each.
    hc = (H // G + 7) // 8
    mfma_flops = float(np.sum((pos.astype(np.float64) + 16) // 16)) * G * hc * (2 * D / 16) * 8192

    def step(ev=None):
        dev.append(L, mem, n_blocks, kn, vn, d_slots)
        if ev is not None:
            ev[0].record(stream)
        dev.attention(L, mem, n_blocks, q, d_blocks, d_tat, d_pos, H, max_pos, out)
        if ev is not None:
            ev[1].record(stream)

    res = {}
    if "decode" in legs:
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        dev.check()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(steps)]
        torch.cuda.synchronize()
        t_start = time.perf_counter()
        for i in range(steps):
            step(evs[i])
        torch.cuda.synchronize()
        wall = time.perf_counter() - t_start
        dev.check()
        attn_ms = float(np.mean([a.elapsed_time(b) for a, b in evs]))
        ms_step = wall * 1e3 / steps
        res.update(ms_per_step=ms_step, tokens_per_s=S / (ms_step / 1e3), attn_ms=attn_ms,
                   attn_gbs=attn_bytes / (attn_ms / 1e3) / 1e9,
                   attn_tflops=flops / (attn_ms / 1e3) / 1e12,
                   attn_mfma_tflops=mfma_flops / (attn_ms / 1e3) / 1e12)
        log(f"[bench] {name} decode step {ms_step:.3f} ms ({S / (ms_step / 1e3):.0f} tok/s); "
            f"attention {attn_ms:.3f} ms = {res['attn_gbs']:.0f} GB/s")

    if cpu and "decode" in legs:
        # Read back the timed step's output before the other legs reuse `out`.
        sample = np.sort(np.random.default_rng(args.seed + 7).choice(items, 8, replace=False))
        got = out[torch.from_numpy(sample).cuda()].cpu().numpy()

    if "layers" in legs:
        # Model order: layer l's append and attention over its S items, layer after layer
        # (items of layer l are rows l*S .. l*S+S-1 of every array above).
        per_layer = []
        for l in range(NL):
            a, b = l * S, (l + 1) * S
            per_layer.append((kn[a:b], vn[a:b], d_slots[a:b], q[a:b], d_tat[a:b], d_pos[a:b],
                              out[a:b]))
        lay_ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(NL)]

        def layer_step(timed=False):
            for l, (k_, v_, s_, q_, t_, p_, o_) in enumerate(per_layer):
                dev.append(L, mem, n_blocks, k_, v_, s_)
                if timed:
                    lay_ev[l][0].record(stream)
                dev.attention(L, mem, n_blocks, q_, d_blocks, t_, p_, H, max_pos, o_)
                if timed:
                    lay_ev[l][1].record(stream)

        for _ in range(warmup):
            layer_step()
        torch.cuda.synchronize()
        dev.check()
        t_start = time.perf_counter()
        for _ in range(steps):
            layer_step()
        torch.cuda.synchronize()
        lwall = (time.perf_counter() - t_start) * 1e3 / steps
        layer_step(timed=True)
        torch.cuda.synchronize()
        dev.check()
        la_ms = float(sum(a.elapsed_time(b) for a, b in lay_ev))
        res.update(layers_ms_per_step=lwall, layers_tokens_per_s=S / (lwall / 1e3),
                   layers_attn_ms=la_ms, layers_attn_gbs=attn_bytes / (la_ms / 1e3) / 1e9)
        log(f"[bench] {name} decode in model order ({NL} x append+attention over {S} items): "
            f"{lwall:.3f} ms/step ({S / (lwall / 1e3):.0f} tok/s); attention {la_ms:.3f} ms = "
            f"{res['layers_attn_gbs']:.0f} GB/s")
        # The same step captured once into a HIP graph and replayed: the device time of the
        # model-order step without this script's per-call launch cost (Python and ctypes
        # issue each call slower than the GPU runs it here).  The replayed outputs must
        # equal the eager step's bit for bit.
        gs = torch.cuda.Stream()
        gs.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(gs):
            layer_step()  # the stream's first launches set up its flag and workspace
        gs.synchronize()
        dev.check(gs)
        eager_out = out.clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=gs):
            layer_step()
        torch.cuda.synchronize()
        for _ in range(max(warmup, 1)):
            graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        dev.check(gs)
        if not torch.equal(out, eager_out):
            raise SystemExit("graph replay of the model-order step differs from the eager step")
        g_ms = e0.elapsed_time(e1) / steps
        res.update(layers_graph_ms_per_step=g_ms, layers_graph_tokens_per_s=S / (g_ms / 1e3),
                   layers_graph_gbs=attn_bytes / (g_ms / 1e3) / 1e9)
        log(f"[bench] {name} model order as one HIP graph: {g_ms:.3f} ms/step "
            f"({S / (g_ms / 1e3):.0f} tok/s; attention bytes / step time = "
            f"{res['layers_graph_gbs']:.0f} GB/s, appends included)")
        del graph

        # The same step with each layer's append inside its attention launch
        # (qvkv_append_attention_async, one launch per layer for f16 pools): the outputs
        # must equal the eager step's bit for bit.
        def fused_step():
            for k_, v_, s_, q_, t_, p_, o_ in per_layer:
                dev.append_attention(L, mem, n_blocks, q_, k_, v_, d_blocks, t_, p_, H,
                                     max_pos, o_)

        out.zero_()
        with torch.cuda.stream(gs):
            fused_step()
        gs.synchronize()
        dev.check(gs)
        if not torch.equal(out, eager_out):
            raise SystemExit("the fused append + attention step differs from the eager step")
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=gs):
            fused_step()
        torch.cuda.synchronize()
        for _ in range(max(warmup, 1)):
            graph.replay()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        dev.check(gs)
        if not torch.equal(out, eager_out):
            raise SystemExit("graph replay of the fused step differs from the eager step")
        f_ms = e0.elapsed_time(e1) / steps
        res.update(layers_fused_ms_per_step=f_ms, layers_fused_tokens_per_s=S / (f_ms / 1e3),
                   layers_fused_gbs=attn_bytes / (f_ms / 1e3) / 1e9)
        log(f"[bench] {name} model order, append fused into attention, one HIP graph: "
            f"{f_ms:.3f} ms/step ({S / (f_ms / 1e3):.0f} tok/s; "
            f"{res['layers_fused_gbs']:.0f} GB/s of attention bytes)")
        del graph, eager_out

    if "gather" in legs:
        # Gather up to 8 layers' items (all positions) into contiguous [G][n][d] per item.
        NGL = min(8, NL)
        gi = S * NGL
        lens = (pos[:gi] + 1).astype(np.uint32)
        out_at = np.concatenate([[0], np.cumsum(lens[:-1], dtype=np.uint64)]).astype(np.uint64)
        tot = int(lens.sum())
        gdt = torch.float16 if dtype == "f16" else torch.float32
        ok = torch.empty(tot * kv_out, dtype=gdt, device="cuda")
        ov = torch.empty_like(ok)
        nt = int(table_at[gi]) if gi < items else blocks.size
        d_gb, d_gl = c32(blocks[:nt]), c32(lens)
        d_go = torch.from_numpy(out_at.view(np.int64)).cuda()
        od = "f16" if dtype == "f16" else "f32"
        g = lambda: dev.gather(L, mem, n_blocks, d_gb, d_tat[:gi], d_gl, d_go,  # noqa: E731
                               int(lens.max()), ok, ov, od)
        timer(g, 2)
        g_ms = timer(g, 5)
        dev.check()
        g_bytes = (tot * kv_out * 2 * bytes_per_value + 2 * ok.numel() * ok.element_size()
                   + nt * 4 + gi * 16)
        res.update(gather_ms=g_ms, gather_gbs=g_bytes / (g_ms / 1e3) / 1e9)
        log(f"[bench] {name} gather {NGL} layers ({od} out): {g_ms:.3f} ms = "
            f"{res['gather_gbs']:.0f} GB/s")
        del ok, ov

    if "copy" in legs:
        # Batched block copy: live blocks into free blocks (the COW / compaction move).
        ncp = min(65536, pool.stats()["free"] - 16)
        src = blocks[:ncp]
        live = np.zeros(n_blocks, bool)
        live[blocks] = True
        dst = np.nonzero(~live)[0][:ncp].astype(np.uint32)
        d_src, d_dst = c32(src), c32(dst)
        cp = lambda: dev.block_copy(L, mem, n_blocks, d_src, d_dst)  # noqa: E731
        timer(cp, 2)
        c_ms = timer(cp, 5)
        dev.check()
        c_bytes = 2.0 * ncp * L.block_bytes + ncp * 8
        res.update(copy_ms=c_ms, copy_gbs=c_bytes / (c_ms / 1e3) / 1e9)
        log(f"[bench] {name} block copy {ncp} blocks: {c_ms:.3f} ms = {res['copy_gbs']:.0f} GB/s")

    if "prefill" in legs:
        # Paged prefill attention: a chunk of PF tokens at the end of every sequence's
        # stored context (positions ctx-1-PF .. ctx-2) on one layer, causal.
        PF = int(min(512, int(ctx.min()) - 1))
        b0, t0_, p0_ = tabs[0]
        seg_pos0 = (p0_.astype(np.int64) - PF).astype(np.uint32)  # p0_ = ctx-1
        n_tok = np.full(S, PF, np.uint32)
        q_at = (np.arange(S, dtype=np.uint32) * PF).astype(np.uint32)
        qp = torch.randn((S * PF, H, D), generator=gen, device="cuda")
        op = torch.empty_like(qp)
        d_pb, d_pt, d_pp, d_qa, d_nt = c32(b0), c32(t0_), c32(seg_pos0), c32(q_at), c32(n_tok)
        pmax = int(seg_pos0.max()) + PF - 1
        pf = lambda: dev.prefill_attention(L, mem, n_blocks, qp, d_pb, d_pt, d_pp,  # noqa: E731
                                           d_qa, d_nt, H, pmax, PF, op)
        timer(pf, 2)
        dev.check()
        p_ms = timer(pf, 5)
        dev.check()
        seen = float(np.sum([PF * (int(p) + 1) + PF * (PF - 1) / 2 for p in seg_pos0]))
        p_flops = 4.0 * H * D * seen
        # MFMA work the f16 prefill kernel issues: per wave (16 query rows) and 32-position
        # tile up to its last row's position, 2*(d/32)*2 + (d/16) v_mfma_f32_16x16x32_f16
        # (q as f16 high part + residual, P as one f16), 8192 FMA each.
        GS = H // G
        rows = PF * GS
        w_first = np.arange(0, rows, 16)
        last_tok = np.minimum(PF - 1, (w_first + 15) // GS)
        tiles = sum(float(np.sum((int(p0) + last_tok + 1 + 31) // 32)) for p0 in seg_pos0) * G
        p_mfma = tiles * (4 * (D // 32) + (D // 16)) * 16384.0
        res.update(prefill_ms=p_ms, prefill_tok_s=S * PF / (p_ms / 1e3),
                   prefill_tflops=p_flops / (p_ms / 1e3) / 1e12)
        if dtype == "f16" and D in (64, 128):  # the LDS-staged 16x16x32 kernel
            res.update(prefill_mfma_tflops=p_mfma / (p_ms / 1e3) / 1e12)
        log(f"[bench] {name} prefill {S} x {PF} tokens (1 layer): {p_ms:.3f} ms = "
            f"{res['prefill_tok_s']:.0f} tok/s, {res['prefill_tflops']:.1f} TFLOP/s")
        del qp, op

    if "prelude" in legs:
        # The attention prelude over one layer's 512-token prefill chunk of every sequence:
        # q/k/v rows in place (bias, QK RMSNorm per head for the Qwen3-like cfg5, else
        # none; RoPE).  Bytes: q, k, v read and written, the RoPE rows read.
        PT = S * 512
        norm = cfg.get("qk_norm", "none")
        xq = torch.randn((PT, H * D), generator=gen, device="cuda")
        xk = torch.randn((PT, kv_out), generator=gen, device="cuda")
        xv = torch.randn((PT, kv_out), generator=gen, device="cuda")
        ang = torch.rand((PT, D // 2), generator=gen, device="cuda") * 6.283
        rope = torch.cat([torch.cos(ang), torch.sin(ang)], dim=1).contiguous()
        qb = torch.randn(H * D, generator=gen, device="cuda")
        kb, vb = (torch.randn(kv_out, generator=gen, device="cuda") for _ in range(2))
        wn = D if norm == "per_head" else None
        qn = torch.rand(wn, generator=gen, device="cuda") + 0.5 if wn else None
        knw = torch.rand(wn, generator=gen, device="cuda") + 0.5 if wn else None
        pre = lambda: dev.prelude(L, H, xq, xk, xv, rope, norm=norm, q_bias=qb,  # noqa: E731
                                  k_bias=kb, v_bias=vb, q_norm=qn, k_norm=knw)
        timer(pre, 2)
        r_ms = timer(pre, 5)
        r_bytes = PT * (H + 2 * G) * D * 4 * 2 + PT * D * 4
        res.update(prelude_ms=r_ms, prelude_gbs=r_bytes / (r_ms / 1e3) / 1e9)
        log(f"[bench] {name} prelude {PT} tokens ({norm} QK norm): {r_ms:.3f} ms = "
            f"{res['prelude_gbs']:.0f} GB/s")
        del xq, xk, xv, rope

    if "calib" in legs:
        # A plain device copy of known size (torch's copy kernel, none of this library's):
        # the reference the PMC traffic summaries scale FETCH_SIZE and WRITE_SIZE by.
        src = torch.empty(1 << 30, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        src.fill_(1.0)
        c_ms = timer(lambda: dst.copy_(src), 3)
        res.update(calib_copy_bytes=2.0 * src.numel() * 4, calib_copy_ms=c_ms)
        log(f"[bench] calibration copy of {src.numel() * 4 / 2**30:.0f} GiB: {c_ms:.3f} ms")
        del src, dst

    if append_ms:
        a_ms = float(np.mean(append_ms))
        a_gbs = float(np.mean(append_bytes)) / (a_ms / 1e3) / 1e9
        res.update(append_ms=a_ms, append_gbs=a_gbs)
        log(f"[bench] {name} bulk append ({CHUNK} tok x {S} seqs x {NL} layers): {a_ms:.3f} ms "
            f"= {a_gbs:.0f} GB/s")

    baseline = None
    if cpu and "decode" in legs:
        baseline = cpu_baseline(args, dev, pool, L, H, blocks, table_at, pos, sample, got,
                                q[torch.from_numpy(sample).cuda()].cpu().numpy(), positions, S,
                                res["ms_per_step"])

    info = dict(cfg=cfg, S=S, NL=NL, G=G, D=D, H=H, B=B, dtype=dtype, ctx=ctx, frag=frag,
                n_blocks=n_blocks, block_bytes=L.block_bytes, attn_bytes=attn_bytes,
                stats=pool.stats(), cpu=baseline)
    del kn, vn, q, out
    pool.close()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res, info


def cpu_baseline(args, dev, pool, L, H, blocks, table_at, pos, sample, got, q, positions_per_step,
                 S, gpu_ms):
    """The reference CPU path restated (oracle, test infrastructure used only as the
    checker and the CPU baseline here): gather through the block table + `attend` per
    (item, head), OpenMP over heads.  Runs on 8 seeded (sequence, layer) items of the
    timed step: their K/V are read back raw from the pool blocks (no GPU kernel involved)
    and decoded from the f16 layout; the GPU's timed output of those items must match
    within the attention tolerance.  Timed for ~cpu_seconds and scaled by positions to one
    whole step."""
    import numpy as np

    import oracle

    G, D, B = L.kv_heads, L.head_dim, L.block
    if L.dtype != "f16":
        return None
    nproc = int(subprocess.run(["nproc"], capture_output=True, text=True).stdout.strip() or 1)
    threads = int(os.environ.get("QVKV_CPU_THREADS", nproc))
    buf = pool.buffer
    bb = L.block_bytes
    ks, vs, lens = [], [], []
    for t in sample:
        n = int(pos[t]) + 1
        ids = blocks[int(table_at[t]):int(table_at[t]) + (n + B - 1) // B]
        raw = np.frombuffer(b"".join(dev.read(buf, int(b) * bb, bb) for b in ids), np.uint16)
        raw = raw.reshape(len(ids), 2, G, B, D)  # per block: K [G][B][d] | V [G][B][d]
        for arr, dst in ((raw[:, 0], ks), (raw[:, 1], vs)):
            rows = arr.transpose(0, 2, 1, 3).reshape(len(ids) * B, G * D)[:n]
            dst.append(rows.view(np.float16).astype(np.float32))
        lens.append(n)
    n_items = len(sample)
    bpl = [(n + B - 1) // B for n in lens]
    nb = int(sum(bpl))
    sim = oracle.SimPool(nb, G, D, B, oracle.F16)
    c_blocks = np.arange(nb, dtype=np.uint32)
    c_tat = np.concatenate([[0], np.cumsum(bpl)[:-1]]).astype(np.uint32)
    c_pos = (np.array(lens) - 1).astype(np.uint32)
    for t in range(n_items):
        p = np.arange(lens[t])
        slots = (c_blocks[c_tat[t] + p // B].astype(np.int64) * B + p % B).astype(np.uint32)
        sim.store(ks[t], vs[t], slots, threads=threads)
    done, positions, t0 = 0, 0, time.perf_counter()
    while True:
        want = sim.attention(q, H, c_blocks, c_tat, c_pos, threads=threads)
        done += n_items
        positions += int(np.sum(c_pos.astype(np.int64) + 1))
        if time.perf_counter() - t0 >= args.cpu_seconds:
            break
    per_position = (time.perf_counter() - t0) / positions
    step_s = per_position * positions_per_step
    tok_s = S / step_s
    diff = got.astype(np.float64) - want
    max_abs = float(np.max(np.abs(diff)))
    rel = float(np.linalg.norm(diff) / np.linalg.norm(want))
    ok = bool(max_abs <= 2e-3 and rel <= 1e-3 and np.isfinite(got).all())
    log(f"[bench] CPU baseline: {per_position * 8192 * 1e3:.1f} ms per 8192 positions on "
        f"{threads} threads -> {step_s:.1f} s per step, {tok_s:.3f} tok/s "
        f"(GPU/CPU {step_s * 1e3 / gpu_ms:.0f}x); timed output of items {sample.tolist()} vs "
        f"the CPU path: max-abs {max_abs:.2e}, rel-L2 {rel:.2e} -> {'ok' if ok else 'MISMATCH'}")
    return {"value": round(tok_s, 4), "unit": "tokens/s", "cores": threads, "nproc": nproc,
            "kind": "port",
            "sample": f"{done} (sequence, layer) item-attentions of gather + attend over "
                      f"{int(c_pos.max()) + 1} positions: 8 seeded items of the timed step "
                      f"(K/V read back raw from their fragmented pool blocks), {H} heads each, "
                      f"scaled by positions to one step ({int(positions_per_step)} positions); "
                      "oracle restatement of SimDevice::attention + math::attend",
            "validation": {"items": sample.tolist(), "max_abs": max_abs, "rel_l2": rel,
                           "tolerance": [2e-3, 1e-3], "ok": ok}}


# --------------------------------------------------------------------------------------
# cfg4: prefix sharing, copy-on-write, LRU eviction, compaction
# --------------------------------------------------------------------------------------

def run_cfg4(args, dev):
    import numpy as np
    import torch

    from qubivex_amd import KvLayout, KvPool

    cfg = CONFIGS["cfg4"]
    NL, G, D, S = cfg["layers"], cfg["kv_heads"], cfg["head_dim"], cfg["seqs"]
    PREFIX, DIV, B = cfg["prefix"], cfg["divergent"], 16
    L = KvLayout("f16", G, D, B)
    bb = L.block_bytes
    need = NL * ((PREFIX + B - 1) // B + S * ((PREFIX % B + DIV + B - 1) // B))
    N = int(need * 1.25) + 64
    pool = KvPool(dev, L, N, NL)
    mem = pool.memory
    stream = torch.cuda.current_stream()
    timer = Timer(torch, stream)
    gen = torch.Generator(device="cuda").manual_seed(args.seed + 4)
    r = np.random.default_rng(args.seed + 4)
    dev.gather_host(L, pool.buffer, [0], [0], [16], [0], 1 << 14)  # grow the staging once
    parent = pool.create()
    for l in range(NL):
        sl = cu32(torch, pool.plan_append([parent], [PREFIX], l))
        k = torch.randn((PREFIX, G * D), generator=gen, device="cuda")
        dev.append(L, mem, N, k, torch.randn_like(k), sl)
    kids = [pool.fork(parent, PREFIX) for _ in range(S)]
    # Divergent appends, every layer in one plan: the first write of each child into the
    # shared partial block copies it (64 children x 32 layers copies of a 64 KiB block, one
    # launch, ordered after the prefix appends above).  GPU time of that launch from the
    # library's own events (qvkv_timing).
    before = dev.transfers()["gpu_ns"]
    slots = pool.plan_append_layers(kids, [DIV] * S, 0, NL)
    cow_ns = dev.transfers()["gpu_ns"] - before
    sl = cu32(torch, slots)
    k = torch.randn((slots.size, G * D), generator=gen, device="cuda")
    v = torch.randn_like(k)
    app_ms = timer(lambda: dev.append(L, mem, N, k, v, sl), 1)
    app_rows = slots.size
    del k, v
    dev.check()
    st = pool.stats()
    cow = st["cow_copies"]
    assert cow == S * NL, st
    # The same copy-on-write batch again, timed over repeated launches with HIP events.
    free = np.zeros(N, bool)
    refs = np.array([pool.refcount(b) for b in range(N)])
    free[refs == 0] = True
    shared = np.nonzero(refs > 1)[0][: S * NL].astype(np.uint32)
    dst = np.nonzero(free)[0][: shared.size].astype(np.uint32)
    d_s, d_d = cu32(torch, shared), cu32(torch, dst)
    bc = lambda: dev.block_copy(L, mem, N, d_s, d_d)  # noqa: E731
    timer(bc, 2)
    bat_ms = timer(bc, 5)
    dev.check()
    # LRU eviction of 25 % of the blocks in use, then compaction under a seeded remap.
    for i in r.permutation(S):
        pool.touch(kids[int(i)])
    used = N - pool.stats()["free"]
    t0 = time.perf_counter()
    released = pool.evict_lru(used // 4)
    evict_s = time.perf_counter() - t0
    comp = {}
    for mode in ("fill", "permute"):
        # "fill": the blocks past the live count into the vacant ids below it (one batch);
        # "permute": every live block under a seeded permutation (dependent batches).
        before = dev.transfers()["gpu_ns"]
        t0 = time.perf_counter()
        moved = pool.compact(seed=args.seed + 44, mode=mode)
        wall = time.perf_counter() - t0
        ns = dev.transfers()["gpu_ns"] - before
        comp[mode] = {"moves": int(moved), "gpu_ms": ns / 1e6, "wall_ms": wall * 1e3,
                      "gbs": 2.0 * moved * bb / ns if ns else None}
    st = pool.stats()
    res = {
        "cow_copies": int(cow), "cow_block_bytes": bb,
        "cow_gbs": 2.0 * cow * bb / cow_ns if cow_ns else None, "cow_us": cow_ns / 1e3,
        "cow_frac": (2.0 * cow * bb / cow_ns if cow_ns else 0) / PEAK_HBM_GBS,
        "cow_batched_ms": bat_ms, "cow_batched_gbs": 2.0 * shared.size * bb / (bat_ms / 1e3) / 1e9,
        "divergent_append_gbs": app_rows * G * D * (8 + 4) / (app_ms / 1e3) / 1e9,
        "evicted_seqs": len(released), "evicted_blocks": int(st["evicted_blocks"]),
        "evict_host_ms": evict_s * 1e3,
        "compaction_moves": comp["fill"]["moves"], "compaction_gpu_ms": comp["fill"]["gpu_ms"],
        "compaction_gbs": comp["fill"]["gbs"], "compaction_wall_ms": comp["fill"]["wall_ms"],
        "compaction_frac": (comp["fill"]["gbs"] or 0) / PEAK_HBM_GBS,
        "compaction_permute": comp["permute"],
    }
    log(f"[bench] cfg4: {cow} COW copies of {bb // 1024} KiB in one launch of the all-layer plan: "
        f"{res['cow_us']:.1f} us ({res['cow_gbs']:.0f} GB/s), repeated {bat_ms:.3f} ms = "
        f"{res['cow_batched_gbs']:.0f} GB/s; evicted {res['evicted_blocks']} blocks; compaction "
        f"(fill) {comp['fill']['moves']} moves in {comp['fill']['gpu_ms']:.3f} ms GPU = "
        f"{comp['fill']['gbs']:.0f} GB/s ({comp['fill']['wall_ms']:.3f} ms wall, planning included); (permute) "
        f"{comp['permute']['moves']} moves in {comp['permute']['gpu_ms']:.3f} ms = "
        f"{comp['permute']['gbs']:.0f} GB/s")
    pool.close()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


# --------------------------------------------------------------------------------------
# cfg1: one sequence, latency-bound
# --------------------------------------------------------------------------------------

def run_cfg1(args, dev):
    import numpy as np
    import torch

    from qubivex_amd import KvLayout, KvPool

    cfg = CONFIGS["cfg1"]
    NL, G, D, H, B = cfg["layers"], cfg["kv_heads"], cfg["head_dim"], cfg["q_heads"], 16
    P, T = cfg["prefill"], cfg["decode"]
    L = KvLayout("f16", G, D, B)
    N = NL * ((P + T) // B + 1) + 64
    pool = KvPool(dev, L, N, NL)
    mem = pool.memory
    gen = torch.Generator(device="cuda").manual_seed(args.seed + 1)
    s = pool.create()
    stream = torch.cuda.current_stream()
    c32 = lambda a: cu32(torch, a)  # noqa: E731
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    sl = c32(np.concatenate([pool.plan_append([s], [P], l) for l in range(NL)]))
    k = torch.randn((NL * P, G * D), generator=gen, device="cuda")
    dev.append(L, mem, N, k, torch.randn_like(k), sl)
    torch.cuda.synchronize()
    prefill_ms = (time.perf_counter() - t0) * 1e3
    q = torch.randn((NL, H, D), generator=gen, device="cuda")
    out = torch.empty_like(q)
    kn = torch.randn((NL, G * D), generator=gen, device="cuda")
    ok = torch.empty(NL * (P + T) * G * D, dtype=torch.float16, device="cuda")
    ov = torch.empty_like(ok)
    # each layer's gathered rows at a fixed stride of P + T positions
    out_at = torch.arange(NL, dtype=torch.int64, device="cuda") * (P + T)
    # the step's tables stay on the device: each sync sends only the ids added at block
    # edges and the positions (one copy, one small kernel)
    tables = pool.device_tables([s], 0, NL, (P + T) // B + 2)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(T)]
    t0 = time.perf_counter()
    for step in range(T):
        # host planning (the runtime's part): every layer's new slot in one call, then the
        # device tables brought up to date
        sl = pool.plan_append_layers([s], [1], 0, NL)
        mp = tables.sync(stream)
        # the device path of one decode step: append, gather and attention of every layer
        # (odd steps: the append inside the attention launch, qvkv_append_attention_async)
        evs[step][0].record(stream)
        if step % 2 == 0:
            dev.append(L, mem, N, kn, kn, c32(sl))
            dev.gather(L, mem, N, tables.blocks, tables.table_at, tables.lens, out_at, mp + 1,
                       ok, ov, "f16")
            dev.attention(L, mem, N, q, tables.blocks, tables.table_at, tables.pos, H, mp, out)
        else:
            dev.append_attention(L, mem, N, q, kn, kn, tables.blocks, tables.table_at,
                                 tables.pos, H, mp, out)
            dev.gather(L, mem, N, tables.blocks, tables.table_at, tables.lens, out_at, mp + 1,
                       ok, ov, "f16")
        evs[step][1].record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    gpu = float(np.mean([a.elapsed_time(b) for a, b in evs[0::2]]))
    gpu_f = float(np.mean([a.elapsed_time(b) for a, b in evs[1::2]]))
    dev.check()
    tables.close()
    pool.close()
    res = {"prefill_append_ms": prefill_ms, "decode_steps": T, "decode_total_ms": wall,
           "decode_step_us": wall / T * 1e3, "decode_step_device_us": gpu * 1e3,
           "decode_step_fused_device_us": gpu_f * 1e3,
           "note": "latency-bound: per step 16 layers x (append 1 + gather + attention); "
                   "decode_step_us includes the Python host planning (one all-layer plan call "
                   "and a sync of device-resident tables per step); decode_step_device_us is "
                   "the three launches from the first to the last (HIP events, even steps), "
                   "decode_step_fused_device_us the two launches with the append inside the "
                   "attention (odd steps); no roofline claim"}
    log(f"[bench] cfg1: prefill-append {P} x {NL} layers {prefill_ms:.2f} ms; {T} decode steps "
        f"(append + gather + attention, all layers) {wall:.1f} ms = {wall / T * 1e3:.0f} us/step "
        f"with host planning, {gpu * 1e3:.1f} us/step on the device ({gpu_f * 1e3:.1f} with the "
        f"append fused into the attention launch)")
    return res


# --------------------------------------------------------------------------------------

def roofline_of(config, res, info):
    if "attn_ms" not in res:
        return None
    return {
        "bound": "hbm",
        "achieved": round(res["attn_gbs"], 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(res["attn_gbs"] / PEAK_HBM_GBS, 4),
        "traffic": traffic_from_profile(config, info["attn_bytes"]),
        "traffic_note": "FETCH_SIZE and WRITE_SIZE per launch from profiles/attention_<cfg>_pmc.json, "
                        "scaled by the copy-kernel calibration there: an estimate",
        "kernel": f"k_attn_mfma<{info['D']},{info['dtype']}>",
        "algorithmic_bytes_per_launch": info["attn_bytes"],
        "avg_launch_ms": round(res["attn_ms"], 4),
    }


def summary(res, info):
    keep = ("ms_per_step", "tokens_per_s", "attn_ms", "attn_gbs", "layers_ms_per_step",
            "layers_tokens_per_s", "layers_attn_gbs", "layers_graph_ms_per_step",
            "layers_graph_tokens_per_s", "layers_graph_gbs", "layers_fused_ms_per_step",
            "layers_fused_tokens_per_s", "layers_fused_gbs", "gather_gbs", "copy_gbs",
            "append_gbs", "prefill_tflops", "prelude_gbs")
    out = {k: round(res[k], 4) for k in keep if k in res}
    for k in ("attn_gbs", "layers_attn_gbs", "layers_graph_gbs", "layers_fused_gbs",
              "gather_gbs", "copy_gbs", "append_gbs"):
        if k in res:
            out[k.replace("_gbs", "_frac")] = round(res[k] / PEAK_HBM_GBS, 4)
    out["workload"] = workload_text(info)
    return out


def workload_text(info):
    cfg, S, ctx = info["cfg"], info["S"], info["ctx"]
    ctx_desc = (f"{S} seqs x {int(ctx[0])} ctx" if (ctx == ctx[0]).all()
                else f"{S} seqs x ctx U[{cfg['ctx'][0]},{cfg['ctx'][1]}] (sum {int(ctx.sum())})")
    return (f"{cfg['name']}: {info['NL']} layers, {info['G']} KV heads, d {info['D']}, "
            f"{info['H']} q heads (GQA {info['H'] // info['G']}:1), {info['dtype']} KV, block "
            f"{info['B']}, {ctx_desc}; step = 1 append/seq/layer + paged decode attention over "
            "all layers")


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); this build has no "
              "multi-GPU path (the paged KV path shards by sequence with no exchange).",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from qubivex_amd import HipDevice

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    torch.cuda.init()
    dev = HipDevice(0)
    log(f"[bench] {dev.describe()}")
    if args.tune:
        from qubivex_amd import kv

        for kvp in args.tune:
            name, value = kvp.split("=")
            kv.tune(name, int(value))
            log(f"[bench] knob {name} = {value}")
    legs = set(args.legs.split(","))
    res, info = run_decode(args.config, args, dev, legs, args.steps, args.warmup,
                           cpu=not args.no_cpu)
    others = {}
    for name in ([] if args.only else [c for c in args.configs.split(",") if c]):
        if name == args.config:
            continue
        if name in DECODE_CONFIGS:
            r2, i2 = run_decode(name, args, dev, {"decode", "layers", "gather", "copy"},
                                max(5, args.steps // 2), 2, cpu=False)
            others[name] = summary(r2, i2)
            others[name]["roofline"] = roofline_of(name, r2, i2)
        elif name == "cfg4":
            others["cfg4"] = run_cfg4(args, dev)
        elif name == "cfg1":
            others["cfg1"] = run_cfg1(args, dev)

    cpu = info["cpu"]
    line = {
        "metric": "paged decode-attn tokens/s at 128x8k (Qwen3-30B-A3B-like KV); "
                  "KV append/gather HBM GB/s",
        "value": round(res.get("tokens_per_s", 0.0), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res.get("ms_per_step", 0.0), 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": info["dtype"],
        "data": "synthetic N(0,1) K/V/Q from a seeded generator; fragmented block tables",
        "config": {
            "workload": workload_text(info),
            "seqs": info["S"], "layers": info["NL"], "kv_heads": info["G"],
            "head_dim": info["D"], "q_heads": info["H"], "block": info["B"],
            "context_positions_per_layer": int(info["ctx"].sum()),
            "pool_blocks": info["n_blocks"],
            "pool_gb": round(info["n_blocks"] * info["block_bytes"] / 1e9, 1),
            "table_discontinuity": round(info["frag"], 3), "seed": args.seed,
        },
        "roofline": roofline_of(args.config, res, info),
        "cpu_baseline": cpu,
        "validated": (cpu or {}).get("validation", {}).get("ok"),
        "legs": {k: round(v, 4) for k, v in res.items()},
        "pool": {k: info["stats"][k] for k in ("blocks", "free", "layers", "synced_rows")},
    }
    if "attn_ms" in res:
        line["model_order"] = {
            "what": "per layer: append + attention over that layer's items, layer after layer",
            "ms_per_step": round(res.get("layers_ms_per_step", 0.0), 4),
            "tokens_per_s": round(res.get("layers_tokens_per_s", 0.0), 1),
            "attention_frac": round(res.get("layers_attn_gbs", 0.0) / PEAK_HBM_GBS, 4),
            "graph_ms_per_step": round(res.get("layers_graph_ms_per_step", 0.0), 4),
            "graph_tokens_per_s": round(res.get("layers_graph_tokens_per_s", 0.0), 1),
            "graph_frac": round(res.get("layers_graph_gbs", 0.0) / PEAK_HBM_GBS, 4),
            "fused_graph_ms_per_step": round(res.get("layers_fused_ms_per_step", 0.0), 4),
            "fused_graph_tokens_per_s": round(res.get("layers_fused_tokens_per_s", 0.0), 1),
            "fused_graph_frac": round(res.get("layers_fused_gbs", 0.0) / PEAK_HBM_GBS, 4),
            "note": "ms_per_step and attention_frac: each call issued from Python (the GPU "
                    "waits on the launches at small batches); graph_*: the same step "
                    "replayed as one HIP graph, appends included in the time; fused_*: "
                    "each layer's append inside its attention launch "
                    "(qvkv_append_attention_async), as one HIP graph",
        }
        line["fraction_of_roofline"] = {
            "attention": round(res["attn_gbs"] / PEAK_HBM_GBS, 4),
            "attention_per_layer": round(res.get("layers_attn_gbs", 0) / PEAK_HBM_GBS, 4),
            "append": round(res.get("append_gbs", 0) / PEAK_HBM_GBS, 4),
            "gather": round(res.get("gather_gbs", 0) / PEAK_HBM_GBS, 4),
            "block_copy": round(res.get("copy_gbs", 0) / PEAK_HBM_GBS, 4),
            "prelude": round(res.get("prelude_gbs", 0) / PEAK_HBM_GBS, 4),
        }
        # MFMA issue rate against the dense f16 peak (2.5 PFLOP/s): decode attention is
        # HBM-bound and uses the matrix cores only for the GQA group contraction.
        line["mfma_utilisation"] = {
            "peak_tflops": PEAK_F16_TFLOPS,
            "attention": round(res["attn_mfma_tflops"] / PEAK_F16_TFLOPS, 4),
            "prefill": round(res.get("prefill_mfma_tflops", 0) / PEAK_F16_TFLOPS, 4),
        }
    if others:
        line["configs"] = others
    print(json.dumps(line), flush=True)
    dev.close()
    if cpu is not None and not cpu["validation"]["ok"]:
        sys.exit(1)  # the timed output does not match the CPU path


def traffic_from_profile(config, algorithmic):
    """HBM bytes per attention launch from the committed rocprofv3 --pmc summary of this
    workload (FETCH_SIZE and WRITE_SIZE scaled by the copy-kernel calibration), when one
    exists for the same algorithmic bytes; else None."""
    path = os.path.join(ROOT, "profiles", f"attention_{config}_pmc.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        p = json.load(f)
    if abs(p.get("algorithmic_bytes", 0) - algorithmic) > 1e-6 * algorithmic:
        return None
    return p.get("traffic_bytes")


if __name__ == "__main__":
    main()
