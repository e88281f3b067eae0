"""Benchmark of the paged KV-cache hot path on one MI355X.

Default workload ("cfg5"): Qwen3-30B-A3B-like KV, 48 layers,
4 KV heads, head_dim 128, 32 query heads (GQA 8:1), f16 storage, block 16, 128 sequences
at 8192 context (~103 GB of KV resident).  Block tables come from the library's pool
manager after seeded alloc/free churn (fragmented).  The pool is filled by bulk
prefill-appends of 512 tokens x all sequences x all layers per call (the timed append leg).

One step = one decode step: one append per sequence on every layer (its newest position)
plus paged decode attention of every query head over the whole context on every layer;
value = tokens/s = sequences / step time.  Inputs are resident in HBM before the timed
region.  Also reported: block-table gather and batched block copy GB/s, and the CPU
baseline: the oracle's restatement of the reference CPU path (gather + `attend`, OpenMP
over heads) on a sample of (sequence, layer) items, scaled to a whole step.

--config cfg2 / cfg3 run the Llama-3-8B-like batched decode (contexts U[256, 4096]) and the
q8_0 configuration (64 x 2048, 1 % x8 outliers) the same way.
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
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="cfg5", choices=sorted(CONFIGS))
    ap.add_argument("--seqs", type=int, default=None, help="override the config's sequences")
    ap.add_argument("--ctx", type=int, default=None, help="override the config's context")
    ap.add_argument("--layers", type=int, default=None, help="override the config's layers")
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--legs", default="append,decode,gather,copy,prefill,prelude")
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
    cfg = dict(CONFIGS[args.config])
    for key in ("seqs", "ctx", "layers"):
        if getattr(args, key) is not None:
            cfg[key] = getattr(args, key)
    dev = HipDevice(0)
    legs = set(args.legs.split(","))
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
    log = lambda *a: print(*a, file=sys.stderr, flush=True)  # noqa: E731
    log(f"[bench] {dev.describe()}; {cfg['name']}; pool {n_blocks} blocks x {L.block_bytes} B = "
        f"{n_blocks * L.block_bytes / 1e9:.1f} GB")
    pool = KvPool(dev, L, n_blocks, NL)
    mem = pool.memory

    def cu32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()

    # ---- seeded churn: scatter the free list before the real sequences allocate
    t0 = time.time()
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
    log(f"[bench] churn: {len(dummies)} sequences, half released ({time.time() - t0:.1f}s)")

    # ---- fill: bulk prefill-append of up to CHUNK tokens per sequence, all layers per call
    CHUNK = 512
    gen = torch.Generator(device="cuda").manual_seed(args.seed)
    stream = torch.cuda.current_stream()
    append_ms, append_bytes = [], []
    fill_to = ctx - 1  # the decode step writes each sequence's position ctx-1
    filled = np.zeros(S, np.int64)
    while (filled < fill_to).any():
        counts = np.minimum(CHUNK, fill_to - filled).astype(np.uint32)
        slots = np.concatenate([pool.plan_append(seqs, counts, l) for l in range(NL)])
        n_rows = slots.size
        sl = cu32(slots)
        k = torch.randn((n_rows, kv_out), generator=gen, device="cuda", dtype=torch.float32)
        v = torch.randn((n_rows, kv_out), generator=gen, device="cuda", dtype=torch.float32)
        if cfg["outliers"]:
            for x in (k, v):
                x[torch.rand(x.shape, generator=gen, device="cuda") < cfg["outliers"]] *= 8.0
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        dev.append(L, mem, n_blocks, k, v, sl)
        e1.record(stream)
        torch.cuda.synchronize()
        dev.check()
        if (counts == CHUNK).all():
            append_ms.append(e0.elapsed_time(e1))
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
    d_slots, d_blocks, d_tat, d_pos = cu32(slots), cu32(blocks), cu32(table_at), cu32(pos)
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
                      attn_gbs=attn_bytes / (attn_ms / 1e3) / 1e9,
                      attn_tflops=flops / (attn_ms / 1e3) / 1e12,
                      attn_mfma_tflops=mfma_flops / (attn_ms / 1e3) / 1e12)
        log(f"[bench] decode step {ms_step:.3f} ms ({S / (ms_step / 1e3):.0f} tok/s); attention "
            f"{attn_ms:.3f} ms = {result['attn_gbs']:.0f} GB/s")

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
        d_gb, d_gl = cu32(blocks[:nt]), cu32(lens)
        d_go = torch.from_numpy(out_at.view(np.int64)).cuda()
        od = "f16" if dtype == "f16" else "f32"
        for _ in range(2):
            dev.gather(L, mem, n_blocks, d_gb, d_tat[:gi], d_gl, d_go, int(lens.max()), ok, ov, od)
        torch.cuda.synchronize()
        reps = 5
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            dev.gather(L, mem, n_blocks, d_gb, d_tat[:gi], d_gl, d_go, int(lens.max()), ok, ov, od)
        e1.record(stream)
        torch.cuda.synchronize()
        dev.check()
        g_ms = e0.elapsed_time(e1) / reps
        g_bytes = (tot * kv_out * 2 * bytes_per_value + 2 * ok.numel() * ok.element_size()
                   + nt * 4 + gi * 16)
        result.update(gather_ms=g_ms, gather_gbs=g_bytes / (g_ms / 1e3) / 1e9)
        log(f"[bench] gather {NGL} layers ({od} out): {g_ms:.3f} ms = {result['gather_gbs']:.0f} GB/s")
        del ok, ov

    if "copy" in legs:
        # Batched block copy: live blocks into free blocks (the COW / compaction move).
        ncp = min(65536, pool.stats()["free"] - 16)
        src = blocks[:ncp]
        live = np.zeros(n_blocks, bool)
        live[blocks] = True
        dst = np.nonzero(~live)[0][:ncp].astype(np.uint32)
        d_src, d_dst = cu32(src), cu32(dst)
        for _ in range(2):
            dev.block_copy(L, mem, n_blocks, d_src, d_dst)
        reps = 5
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(reps):
            dev.block_copy(L, mem, n_blocks, d_src, d_dst)
        e1.record(stream)
        torch.cuda.synchronize()
        dev.check()
        c_ms = e0.elapsed_time(e1) / reps
        c_bytes = 2.0 * ncp * L.block_bytes + ncp * 8
        result.update(copy_ms=c_ms, copy_gbs=c_bytes / (c_ms / 1e3) / 1e9)
        log(f"[bench] block copy {ncp} blocks: {c_ms:.3f} ms = {result['copy_gbs']:.0f} GB/s")

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
        d_pb, d_pt, d_pp, d_qa, d_nt = cu32(b0), cu32(t0_), cu32(seg_pos0), cu32(q_at), cu32(n_tok)
        pmax = int(seg_pos0.max()) + PF - 1
        for _ in range(2):
            dev.prefill_attention(L, mem, n_blocks, qp, d_pb, d_pt, d_pp, d_qa, d_nt, H, pmax, PF, op)
        torch.cuda.synchronize()
        dev.check()
        reps = 5
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            dev.prefill_attention(L, mem, n_blocks, qp, d_pb, d_pt, d_pp, d_qa, d_nt, H, pmax, PF, op)
        e1.record(stream)
        torch.cuda.synchronize()
        dev.check()
        p_ms = e0.elapsed_time(e1) / reps
        seen = float(np.sum([PF * (int(p) + 1) + PF * (PF - 1) / 2 for p in seg_pos0]))
        p_flops = 4.0 * H * D * seen
        # MFMA work the f16 prefill kernel issues: per wave (16 query rows) and 32-position
        # tile up to its last row's position, 2*(d/32)*2 + (d/16)*2 v_mfma_f32_16x16x32_f16
        # (q and p as f16 high part + residual), 8192 FMA each.
        GS = H // G
        rows = PF * GS
        w_first = np.arange(0, rows, 16)
        last_tok = np.minimum(PF - 1, (w_first + 15) // GS)
        tiles = sum(float(np.sum((int(p0) + last_tok + 1 + 31) // 32)) for p0 in seg_pos0) * G
        p_mfma = tiles * (4 * (D // 32) + 2 * (D // 16)) * 16384.0
        result.update(prefill_ms=p_ms, prefill_tok_s=S * PF / (p_ms / 1e3),
                      prefill_tflops=p_flops / (p_ms / 1e3) / 1e12)
        if dtype == "f16" and D in (64, 128):  # the LDS-staged 16x16x32 kernel
            result.update(prefill_mfma_tflops=p_mfma / (p_ms / 1e3) / 1e12)
        log(f"[bench] prefill {S} x {PF} tokens (1 layer, ctx {int(ctx.min())}..{int(ctx.max())}): "
            f"{p_ms:.3f} ms = {result['prefill_tok_s']:.0f} tok/s, {result['prefill_tflops']:.1f} TFLOP/s")
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
        kn = torch.rand(wn, generator=gen, device="cuda") + 0.5 if wn else None

        def pre():
            dev.prelude(L, H, xq, xk, xv, rope, norm=norm, q_bias=qb, k_bias=kb, v_bias=vb,
                        q_norm=qn, k_norm=kn)
        for _ in range(2):
            pre()
        torch.cuda.synchronize()
        reps = 5
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            pre()
        e1.record(stream)
        torch.cuda.synchronize()
        r_ms = e0.elapsed_time(e1) / reps
        r_bytes = PT * (H + 2 * G) * D * 4 * 2 + PT * D * 4
        result.update(prelude_ms=r_ms, prelude_gbs=r_bytes / (r_ms / 1e3) / 1e9)
        log(f"[bench] prelude {PT} tokens ({norm} QK norm): {r_ms:.3f} ms = "
            f"{result['prelude_gbs']:.0f} GB/s")
        del xq, xk, xv, rope

    if append_ms:
        a_ms = float(np.mean(append_ms))
        a_gbs = float(np.mean(append_bytes)) / (a_ms / 1e3) / 1e9
        result.update(append_ms=a_ms, append_gbs=a_gbs)
        log(f"[bench] bulk append ({CHUNK} tok x {S} seqs x {NL} layers): {a_ms:.3f} ms = {a_gbs:.0f} GB/s")

    cpu = None
    if not args.no_cpu and "decode" in legs:
        cpu = cpu_baseline(args, dtype, G, D, H, B, int(ctx.max()), positions, S,
                           result["ms_per_step"], log)

    stats = pool.stats()
    ctx_desc = (f"{S} seqs x {int(ctx[0])} ctx" if (ctx == ctx[0]).all()
                else f"{S} seqs x ctx U[{cfg['ctx'][0]},{cfg['ctx'][1]}] (sum {int(ctx.sum())})")
    line = {
        "metric": "paged decode-attn tokens/s at 128x8k (Qwen3-30B-A3B-like KV); "
                  "KV append/gather HBM GB/s",
        "value": round(result.get("tokens_per_s", 0.0), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(result.get("ms_per_step", 0.0), 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic N(0,1) K/V/Q from a seeded generator; fragmented block tables",
        "config": {
            "workload": f"{cfg['name']}: {NL} layers, {G} KV heads, d {D}, {H} q heads "
                        f"(GQA {H // G}:1), {dtype} KV, block {B}, {ctx_desc}; step = 1 append/"
                        "seq/layer + paged decode attention over all layers",
            "seqs": S, "layers": NL, "kv_heads": G, "head_dim": D, "q_heads": H, "block": B,
            "context_positions_per_layer": int(ctx.sum()), "pool_blocks": n_blocks,
            "pool_gb": round(n_blocks * L.block_bytes / 1e9, 1),
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
            "traffic": traffic_from_profile(args.config, attn_bytes),
            "kernel": f"k_attn_mfma<{D},{'q8_0' if dtype == 'q8_0' else 'f16'}>",
            "algorithmic_bytes_per_launch": attn_bytes,
            "avg_launch_ms": round(result["attn_ms"], 4),
        }
        line["fraction_of_roofline"] = {
            "attention": round(result["attn_gbs"] / PEAK_HBM_GBS, 4),
            "append": round(result.get("append_gbs", 0) / PEAK_HBM_GBS, 4),
            "gather": round(result.get("gather_gbs", 0) / PEAK_HBM_GBS, 4),
            "block_copy": round(result.get("copy_gbs", 0) / PEAK_HBM_GBS, 4),
            "prelude": round(result.get("prelude_gbs", 0) / PEAK_HBM_GBS, 4),
        }
        # MFMA issue rate against the dense f16 peak (2.5 PFLOP/s): decode attention is
        # HBM-bound and uses the matrix cores only for the GQA group contraction.
        line["mfma_utilisation"] = {
            "peak_tflops": PEAK_F16_TFLOPS,
            "attention": round(result["attn_mfma_tflops"] / PEAK_F16_TFLOPS, 4),
            "prefill": round(result.get("prefill_mfma_tflops", 0) / PEAK_F16_TFLOPS, 4),
        }
    print(json.dumps(line), flush=True)
    pool.close()
    dev.close()


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


def cpu_baseline(args, dtype, G, D, H, B, CTX, positions_per_step, S, gpu_ms, log):
    """The reference CPU path restated (oracle): gather through the block table + `attend`
    per (item, head), OpenMP over heads, on a sample of (sequence, layer) items at CTX
    positions; scaled by positions to one whole step."""
    import numpy as np

    import oracle

    threads = int(os.environ.get("QVKV_CPU_THREADS", min(16, os.cpu_count() or 1)))
    n_items = 16
    r = np.random.default_rng(args.seed + 1)
    bpl = (CTX + B - 1) // B
    nb = n_items * bpl
    sim = oracle.SimPool(nb, G, D, B, oracle.F16 if dtype == "f16" else oracle.Q8_0)
    blocks = r.permutation(nb).astype(np.uint32)
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
    per_position = (time.perf_counter() - t0) / (done * CTX)
    step_s = per_position * positions_per_step
    tok_s = S / step_s
    log(f"[bench] CPU baseline: {per_position * CTX * 1e3:.1f} ms per {CTX}-position item on "
        f"{threads} threads -> {step_s:.1f} s per step, {tok_s:.3f} tok/s "
        f"(GPU/CPU {step_s * 1e3 / gpu_ms:.0f}x)")
    return {"value": round(tok_s, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{done} (sequence, layer) items of gather + attend over {CTX} positions "
                      f"({n_items} distinct, {H} heads each), scaled by positions to one step "
                      f"({int(positions_per_step)} positions); oracle restatement of "
                      "SimDevice::attention + math::attend"}


if __name__ == "__main__":
    main()
