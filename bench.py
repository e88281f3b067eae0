"""Benchmark of the paged KV-cache hot path on one MI355X.

Workload ("cfg5"): Qwen3-30B-A3B-like KV, 48 layers, 4 KV heads,
head_dim 128, 32 query heads (GQA 8:1), f16 storage, block 16, 128 sequences at 8192
context (~103 GB of KV resident).  Block tables come from the library's pool manager
after seeded alloc/free churn (fragmented).  The pool is filled by bulk prefill-appends
of 512 tokens x 128 sequences x 48 layers per call (timed: the append leg).

One step = one decode step: one append per sequence on every layer (position 8191) plus
paged decode attention of 32 heads over positions 0..8191 on every layer; the value is
tokens/s = 128 / step time.  Inputs are resident in HBM before the timed region.

Also reported: block-table gather (f16 -> f16) and batched block copy GB/s, and the CPU
baseline: the oracle's restatement of the reference CPU path (gather + `attend`, OpenMP
over heads) on a sample of (sequence, layer) items, scaled to a whole step.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seqs", type=int, default=128)
    ap.add_argument("--ctx", type=int, default=8192)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--legs", default="append,decode,gather,copy")
    ap.add_argument("--dtype", default="f16", choices=["f16", "q8_0"])
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); this build has no "
              "multi-GPU path (the paged KV path shards by sequence with no exchange).",
              file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    from qubivex_amd import HipDevice, KvLayout, KvPool

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    torch.cuda.init()
    dev = HipDevice(0)
    legs = set(args.legs.split(","))
    S, CTX, NL = args.seqs, args.ctx, args.layers
    G, D, H, B = 4, 128, 32, 16
    L = KvLayout(args.dtype, G, D, B)
    kv_out = G * D
    bpl = (CTX + B - 1) // B  # blocks per (sequence, layer)
    real_blocks = S * NL * bpl
    n_blocks = int(real_blocks * 1.25) + 1024
    log = lambda *a: print(*a, file=sys.stderr, flush=True)  # noqa: E731
    log(f"[bench] {dev.describe()}; pool {n_blocks} blocks x {L.block_bytes} B = "
        f"{n_blocks * L.block_bytes / 1e9:.1f} GB")
    pool = KvPool(dev, L, n_blocks, NL)
    pool_ptr = pool.ptr

    def cu32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()

    class Raw:  # a device pointer in the shape the bindings take
        def __init__(self, p):
            self.p = p

        def data_ptr(self):
            return self.p

    praw = Raw(pool_ptr)

    # ---- seeded churn: scatter the free list before the real sequences allocate
    r = np.random.default_rng(args.seed)
    t0 = time.time()
    dummies = []
    budget = int(n_blocks * 0.2)
    used = 0
    while used < budget:
        s = pool.create()
        layer = int(r.integers(NL))
        n = int(r.integers(16, 16 * 64))
        pool.plan_append([s], [n], layer)
        used += (n + B - 1) // B
        dummies.append(s)
    order = r.permutation(len(dummies))
    for i in order[: len(order) // 2]:
        pool.release(dummies[i])
    keep = [dummies[i] for i in order[len(order) // 2:]]
    seqs = [pool.create() for _ in range(S)]
    log(f"[bench] churn: {len(dummies)} sequences, half released ({time.time() - t0:.1f}s)")

    # ---- fill: bulk prefill-append of CHUNK tokens x S sequences x NL layers per call
    CHUNK = 512
    gen = torch.Generator(device="cuda").manual_seed(args.seed)
    append_ms, append_bytes = [], []
    filled = 0
    fill_to = CTX - 1  # the decode step writes position CTX-1
    stream = torch.cuda.current_stream()
    while filled < fill_to:
        c = min(CHUNK, fill_to - filled)
        slots = np.concatenate([pool.plan_append(seqs, [c] * S, l) for l in range(NL)])
        n_rows = slots.size
        sl = cu32(slots)
        k = torch.randn((n_rows, kv_out), generator=gen, device="cuda", dtype=torch.float32)
        v = torch.randn((n_rows, kv_out), generator=gen, device="cuda", dtype=torch.float32)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        dev.append(L, praw, n_blocks, k, v, sl)
        e1.record(stream)
        torch.cuda.synchronize()
        dev.check()
        if c == CHUNK:
            append_ms.append(e0.elapsed_time(e1))
            append_bytes.append(n_rows * kv_out * (4 * 2 + 2 * (2 if args.dtype == "f16" else 34 / 32))
                                + n_rows * 4)
        filled += c
        del k, v, sl
    for s in keep:
        pool.release(s)
    log(f"[bench] filled {fill_to} positions x {S} seqs x {NL} layers ({time.time() - t0:.1f}s)")

    # ---- the decode step's inputs: one new token per (sequence, layer) at position CTX-1
    slots = np.concatenate([pool.plan_append(seqs, [1] * S, l) for l in range(NL)])
    tabs = [pool.tables(seqs, l) for l in range(NL)]
    blocks = np.concatenate([t[0] for t in tabs])
    offs = np.cumsum([0] + [t[0].size for t in tabs[:-1]])
    table_at = np.concatenate([t[1] + o for t, o in zip(tabs, offs)]).astype(np.uint32)
    pos = np.concatenate([t[2] for t in tabs]).astype(np.uint32)
    items = pos.size
    assert items == S * NL and int(pos.max()) == CTX - 1 and int(pos.min()) == CTX - 1
    frag = float(np.mean(np.diff(blocks.astype(np.int64)) != 1))
    d_slots, d_blocks, d_tat, d_pos = cu32(slots), cu32(blocks), cu32(table_at), cu32(pos)
    kn = torch.randn((items, kv_out), generator=gen, device="cuda")
    vn = torch.randn((items, kv_out), generator=gen, device="cuda")
    q = torch.randn((items, H, D), generator=gen, device="cuda")
    out = torch.empty((items, H, D), device="cuda")
    max_pos = int(pos.max())
    kv_bytes_step = float(np.sum(pos.astype(np.float64) + 1)) * kv_out * 2 * (
        2 if args.dtype == "f16" else 34 / 32)
    attn_bytes = (kv_bytes_step + q.numel() * 4 * 2 + blocks.size * 4 + items * 8)
    flops = 4.0 * H * D * float(np.sum(pos.astype(np.float64) + 1))

    def step(ev=None):
        dev.append(L, praw, n_blocks, kn, vn, d_slots)
        if ev is not None:
            ev[0].record(stream)
        dev.attention(L, praw, n_blocks, q, d_blocks, d_tat, d_pos, H, max_pos, out)
        if ev is not None:
            ev[1].record(stream)

    result = {}
    if "decode" in legs:
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        dev.check()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(args.steps)]
        torch.cuda.synchronize()
        t_start = time.perf_counter()
        for i in range(args.steps):
            step(evs[i])
        torch.cuda.synchronize()
        wall = time.perf_counter() - t_start
        dev.check()
        attn_ms = float(np.mean([a.elapsed_time(b) for a, b in evs]))
        ms_step = wall * 1e3 / args.steps
        result.update(ms_per_step=ms_step, tokens_per_s=S / (ms_step / 1e3), attn_ms=attn_ms,
                      attn_gbs=attn_bytes / (attn_ms / 1e3) / 1e9, attn_tflops=flops / (attn_ms / 1e3) / 1e12)
        log(f"[bench] decode step {ms_step:.3f} ms ({S / (ms_step / 1e3):.0f} tok/s); attention "
            f"{attn_ms:.3f} ms = {result['attn_gbs']:.0f} GB/s")

    if "gather" in legs:
        # Gather NG layers' items (all positions) into contiguous f16 [G][n][d] per item.
        NGL = min(8, NL)
        gi = S * NGL
        lens = (pos[:gi] + 1).astype(np.uint32)
        out_at = np.concatenate([[0], np.cumsum(lens[:-1], dtype=np.uint64)]).astype(np.uint64)
        tot = int(lens.sum())
        gdt = torch.float16 if args.dtype == "f16" else torch.float32
        ok = torch.empty(tot * kv_out, dtype=gdt, device="cuda")
        ov = torch.empty_like(ok)
        nt = int(table_at[gi]) if gi < items else blocks.size
        d_gb = cu32(blocks[:nt])
        d_gl = cu32(lens)
        d_go = torch.from_numpy(out_at.view(np.int64)).cuda()
        od = "f16" if args.dtype == "f16" else "f32"
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(2):
            dev.gather(L, praw, n_blocks, d_gb, d_tat[:gi], d_gl, d_go, int(lens.max()), ok, ov, od)
        torch.cuda.synchronize()
        reps = 5
        e0.record(stream)
        for _ in range(reps):
            dev.gather(L, praw, n_blocks, d_gb, d_tat[:gi], d_gl, d_go, int(lens.max()), ok, ov, od)
        e1.record(stream)
        torch.cuda.synchronize()
        dev.check()
        g_ms = e0.elapsed_time(e1) / reps
        g_bytes = tot * kv_out * 2 * (2 if args.dtype == "f16" else 34 / 32) + \
            2 * ok.numel() * ok.element_size() + nt * 4 + gi * 16
        result.update(gather_ms=g_ms, gather_gbs=g_bytes / (g_ms / 1e3) / 1e9)
        log(f"[bench] gather {NGL} layers: {g_ms:.3f} ms = {result['gather_gbs']:.0f} GB/s")
        del ok, ov

    if "copy" in legs:
        # Batched block copy: 65536 live blocks into free blocks (COW / compaction moves).
        st = pool.stats()
        ncp = min(65536, st["free"] - 16)
        src = blocks[:ncp]
        live = np.zeros(n_blocks, bool)
        live[blocks] = True
        dst = np.nonzero(~live)[0][:ncp].astype(np.uint32)
        d_src, d_dst = cu32(src), cu32(dst)
        for _ in range(2):
            dev.block_copy(L, praw, n_blocks, d_src, d_dst)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 5
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(reps):
            dev.block_copy(L, praw, n_blocks, d_src, d_dst)
        e1.record(stream)
        torch.cuda.synchronize()
        dev.check()
        c_ms = e0.elapsed_time(e1) / reps
        c_bytes = 2.0 * ncp * L.block_bytes + ncp * 8
        result.update(copy_ms=c_ms, copy_gbs=c_bytes / (c_ms / 1e3) / 1e9)
        log(f"[bench] block copy {ncp} blocks: {c_ms:.3f} ms = {result['copy_gbs']:.0f} GB/s")

    if append_ms:
        a_ms = float(np.mean(append_ms))
        a_gbs = float(np.mean(append_bytes)) / (a_ms / 1e3) / 1e9
        result.update(append_ms=a_ms, append_gbs=a_gbs)
        log(f"[bench] bulk append ({CHUNK} tok x {S} seqs x {NL} layers): {a_ms:.3f} ms = {a_gbs:.0f} GB/s")

    cpu = None
    if not args.no_cpu and "decode" in legs:
        cpu = cpu_baseline(args, G, D, H, B, CTX, S * NL, S, result["ms_per_step"], log)

    stats = pool.stats()
    line = {
        "metric": "paged decode-attn tokens/s at 128x8k (Qwen3-30B-A3B-like KV); KV append/gather HBM GB/s",
        "value": round(result.get("tokens_per_s", 0.0), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(result.get("ms_per_step", 0.0), 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic N(0,1) K/V/Q from a seeded generator; fragmented block tables",
        "config": {
            "workload": f"cfg5: {NL} layers, {G} KV heads, d {D}, {H} q heads (GQA {H // G}:1), "
                        f"{args.dtype} KV, block {B}, {S} seqs x {CTX} ctx; step = 1 append/seq/layer "
                        "+ paged decode attention over all layers",
            "seqs": S, "ctx": CTX, "layers": NL, "kv_heads": G, "head_dim": D, "q_heads": H,
            "block": B, "pool_blocks": n_blocks, "pool_gb": round(n_blocks * L.block_bytes / 1e9, 1),
            "table_discontinuity": round(frag, 3), "seed": args.seed,
        },
        "roofline": None,
        "cpu_baseline": cpu,
        "legs": {k: round(v, 4) for k, v in result.items()},
        "pool": {k: stats[k] for k in ("blocks", "free", "layers", "synced_rows")},
    }
    if "attn_ms" in result:
        line["roofline"] = {
            "bound": "hbm",
            "achieved": round(result["attn_gbs"], 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(result["attn_gbs"] / PEAK_HBM_GBS, 4),
            "traffic": None,
            "kernel": "k_attn_mfma<128,false>",
            "algorithmic_bytes_per_launch": attn_bytes,
            "avg_launch_ms": round(result["attn_ms"], 4),
        }
        line["fraction_of_roofline"] = {
            "attention": round(result["attn_gbs"] / PEAK_HBM_GBS, 4),
            "append": round(result.get("append_gbs", 0) / PEAK_HBM_GBS, 4),
            "gather": round(result.get("gather_gbs", 0) / PEAK_HBM_GBS, 4),
            "block_copy": round(result.get("copy_gbs", 0) / PEAK_HBM_GBS, 4),
        }
    print(json.dumps(line), flush=True)
    pool.close()
    dev.close()


def cpu_baseline(args, G, D, H, B, CTX, items_per_step, S, gpu_ms, log):
    """The reference CPU path restated (oracle): gather through the block table + `attend`
    per (item, head), OpenMP over heads, on a sample of (sequence, layer) items at the full
    context; scaled to one whole step (items_per_step items)."""
    import numpy as np

    import oracle

    threads = int(os.environ.get("QVKV_CPU_THREADS", min(16, os.cpu_count() or 1)))
    n_items = 16
    r = np.random.default_rng(args.seed + 1)
    bpl = (CTX + B - 1) // B
    nb = n_items * bpl
    sim = oracle.SimPool(nb, G, D, B, oracle.F16 if args.dtype == "f16" else oracle.Q8_0)
    ids = r.permutation(nb).astype(np.uint32)
    blocks = ids
    table_at = (np.arange(n_items) * bpl).astype(np.uint32)
    pos = np.full(n_items, CTX - 1, np.uint32)
    for t in range(n_items):
        p = np.arange(CTX)
        slots = (blocks[table_at[t] + p // B].astype(np.int64) * B + p % B).astype(np.uint32)
        k = r.standard_normal((CTX, G * D), dtype=np.float32)
        v = r.standard_normal((CTX, G * D), dtype=np.float32)
        sim.store(k, v, slots, threads=threads)
    q = r.standard_normal((n_items, H, D), dtype=np.float32)
    done, t0 = 0, time.perf_counter()
    while True:
        sim.attention(q, H, blocks, table_at, pos, threads=threads)
        done += n_items
        if time.perf_counter() - t0 >= args.cpu_seconds:
            break
    per_item = (time.perf_counter() - t0) / done
    step_s = per_item * items_per_step
    tok_s = S / step_s
    log(f"[bench] CPU baseline: {per_item * 1e3:.1f} ms per (seq, layer) item on {threads} threads "
        f"-> {step_s:.1f} s per step, {tok_s:.2f} tok/s (GPU/CPU {step_s * 1e3 / gpu_ms:.0f}x)")
    return {"value": round(tok_s, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{done} (sequence, layer) items of gather + attend over {CTX} positions "
                      f"({n_items} distinct, {H} heads each), scaled x{items_per_step}/item to one "
                      "step; oracle restatement of SimDevice::attention + math::attend"}


if __name__ == "__main__":
    main()
