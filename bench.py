#!/usr/bin/env python3
"""Batch-1 greedy decode throughput of the gfx950 Granite-MoE engine on one GPU.

Workload: Granite-3B-A800M shape (32 layers, hidden 1536, 24 query / 8 KV heads of 64, 40 experts top-8 with ffn
512, vocab 49155), random-init weights N(0, 0.02) quantised to Q8_0 (tied head too), fp32 norms, fp16 KV cache
pre-filled with N(0, 1) to 4096 positions. A step is one decode token (the whole model, greedy argmax on the
device); the timed region replays the captured step graph K times with the token fed back on the device.

Prints one JSON line: tok/s, the HBM roofline of the dominant kernel (HIP events around its launches on the
engine's stream) and, as the CPU baseline, the decode rate on this host of a C++ port of the reference's CPU path
(oracle/cpu_port.cpp).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "lastro-rust_amd"))

HBM_PEAK_GBS = 8000.0
CTX = 4096


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def kernel_bytes(kind, cfg, ctx, wd, ed, nsplit):
    """Algorithmic HBM bytes of one launch of a kernel class at `ctx` cached positions: the weights it must stream
    (only the k routed experts for the expert kernels), the KV it must read and the split partials the attention
    kernels exchange; other activations are < 0.1% of a layer's bytes and left out. The output projection also reads
    the router's columns of its rows (for the MoE-norm partials of its epilogue) and the router kernel reads those
    partials instead of the router."""
    import moert
    H, d, I = cfg.hidden, cfg.head_dim, cfg.inter
    qd, kvd = cfg.heads * d, cfg.kv_heads * d
    b = moert.dtype_bytes
    return {
        moert.K_EMBED: b(ed, H),
        moert.K_QKV: b(wd, (qd + 2 * kvd) * H),
        moert.K_ATTN_SPLIT: 2 * kvd * 2 * ctx,
        moert.K_ATTN_COMBINE: cfg.heads * nsplit * 66 * 4,
        moert.K_OPROJ: b(wd, H * qd) + b(wd, cfg.experts * H),
        moert.K_ROUTE_UP: 65 * 256 * 4 + cfg.top_k * b(wd, 2 * I * H),
        moert.K_EXPERT_DOWN: cfg.top_k * b(wd, H * I),
        moert.K_HEAD: b(ed, cfg.vocab * H),
        moert.K_HEAD_ARGMAX: 0,
        # q/k/v weights and the KV it reads; its queries and split partials stay in the L2 of their XCD
        moert.K_ATTN_BLOCK: b(wd, (qd + 2 * kvd) * H) + 2 * kvd * 2 * ctx,
        # the MoE-norm partials, the k routed experts' gate/up and down rows, the down outputs it leaves
        moert.K_MOE_XCD: 65 * 256 * 4 + cfg.top_k * b(wd, 3 * I * H) + cfg.top_k * H * 4,
        moert.K_MOE_COMBINE: 0,
        # a whole layer: q/k/v and the KV it reads, the output projection, the router rows, the k routed experts;
        # its exchanges stay in the XCDs' L2s or are a few KB device-wide
        moert.K_LAYER: b(wd, (qd + 2 * kvd) * H) + 2 * kvd * 2 * ctx + b(wd, H * qd) + b(wd, cfg.experts * H)
        + cfg.top_k * b(wd, 3 * I * H),
        moert.K_LAYER_COMBINE: 0,
    }[kind]


def measured_traffic(kernel):
    """HBM bytes per launch of `k_<kernel>` from the committed FETCH_SIZE/WRITE_SIZE summary (calibrated against a
    copy of known size); None when the summary has no row for it."""
    path = os.path.join(ROOT, "profiles", "decode3b_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 5 and cells[0] == f"k_{kernel}":
            return int(cells[4])
    return None


def prefill_block(g, cfg, seed, ctx, decode_tok_s, m=32, reps=5):
    """Multi-position step of the whole model: m positions appended after ctx cached ones in one
    moert_step_batched call (bit-identical to m decode steps); the best of `reps` host-timed calls, each with its
    own synchronisation."""
    import numpy as np
    toks = np.random.default_rng(seed + 7).integers(0, cfg.vocab, m)

    def timed():
        g.set_position(ctx)
        g.step_batched(toks, want_logits=False)
        best = None
        for _ in range(reps):
            g.set_position(ctx)
            t0 = time.perf_counter()
            g.step_batched(toks, want_logits=False)
            t = time.perf_counter() - t0
            best = t if best is None else min(best, t)
        return best

    best = timed()
    log(f"multi-position step of {m} at {ctx}: {best * 1e3:.2f} ms, {m / best:.0f} tok/s "
        f"({m / best / decode_tok_s:.2f}x the decode loop)")
    out = {"positions": m, "context": ctx, "ms_per_block": round(best * 1e3, 3), "tok_s": round(m / best, 1),
           "vs_decode": round(m / best / decode_tok_s, 2)}
    # the same block with the experts through the grouped int8 MFMA kernels (moert_batched_mode 1)
    g.batched_mode(1)
    gbest = timed()
    g.batched_mode(0)
    log(f"multi-position step of {m} at {ctx}, grouped experts: {gbest * 1e3:.2f} ms, {m / gbest:.0f} tok/s")
    out["grouped"] = {"ms_per_block": round(gbest * 1e3, 3), "tok_s": round(m / gbest, 1),
                      "vs_decode": round(m / gbest / decode_tok_s, 2)}
    return out


def batched_step(cfg, seed, iters, m=16, nblocks=4):
    """16 positions through one MoE block of the 3B shape at once (router + top-8 per position with the Zipf(1.1)
    router bias, experts regrouped into the grouped int8 MFMA GEMM), rotating over `nblocks` blocks of separate
    weights (400 MB of experts, beyond the 256 MB last-level cache). Reports the block step time, its kernels, the
    expert bytes it must stream (U distinct experts x 2,506,752 B + router) and the per-position GEMV path timed on
    the same blocks for comparison."""
    import numpy as np

    import moert
    H, I, E, k = cfg.hidden, cfg.inter, cfg.experts, cfg.top_k
    blocks, uniq = [], []
    for b in range(nblocks):
        router = moert.synth_quantized(seed + b, 900, E * H, 0.02, moert.Q8_0)
        gu = moert.synth_quantized(seed + b, 901, E * 2 * I * H, 0.02, moert.Q8_0)
        dn = moert.synth_quantized(seed + b, 902, E * H * I, 0.02, moert.Q8_0)
        blk = moert.GpuBlock(H, I, E, k, router, gu, dn, moert.Q8_0, router_bias=moert.zipf_bias(E, seed + b))
        x = moert.synth_normal(seed + b, 903, m * H).reshape(m, H)
        blk.forward_batched(x)
        uniq.append(blk.experts_in_step())
        blocks.append(blk)
    t = moert.time_batched(blocks, m, iters)
    # the same step as one launch of 256 workgroups (moert_block_batched_kernel 1), where the device allows it
    one = None
    try:
        for blk in blocks:
            blk.batched_kernel(1)
        t1 = moert.time_batched(blocks, m, iters)
        one = {"block_step_us": round(t1["step"], 2), "launch_us": round(t1["launch"], 2)}
    except moert.MoertError as exc:
        one = {"skipped": str(exc)}
    for blk in blocks:
        blk.batched_kernel(0)
    per_pos_us = blocks[0].time(max(4, iters)) * m
    for blk in blocks:
        blk.close()
    u_mean = sum(uniq) / len(uniq)
    expert_bytes = moert.dtype_bytes(moert.Q8_0, 3 * I * H)
    nbytes = u_mean * expert_bytes + moert.dtype_bytes(moert.Q8_0, E * H)
    gu_bytes = u_mean * moert.dtype_bytes(moert.Q8_0, 2 * I * H)
    dn_bytes = u_mean * moert.dtype_bytes(moert.Q8_0, I * H)
    flops = 2 * m * k * 3 * I * H
    out = {"positions": m, "experts_distinct_mean": u_mean, "block_step_us": round(t["step"], 2),
           "kernels_us": {key: round(t[key], 2) for key in ("route", "up", "down", "combine")},
           "bytes": int(nbytes), "achieved_gbs": round(nbytes / (t["step"] * 1e-6) / 1e9, 1),
           "up_gbs": round(gu_bytes / (t["up"] * 1e-6) / 1e9, 1),
           "down_gbs": round(dn_bytes / (t["down"] * 1e-6) / 1e9, 1),
           "useful_tops": round(flops / ((t["up"] + t["down"]) * 1e-6) / 1e12, 3),
           "per_position_path_us": round(per_pos_us, 2),
           "speedup_vs_per_position": round(per_pos_us / t["step"], 2),
           "one_launch": one}
    if "block_step_us" in one:
        one["achieved_gbs"] = round(nbytes / (one["block_step_us"] * 1e-6) / 1e9, 1)
    log(f"batched step m={m}: {t['step']:.1f} us per block ({u_mean:.1f} experts, {out['achieved_gbs']} GB/s), "
        f"one launch {one.get('block_step_us', '-')} us, per-position path {per_pos_us:.1f} us")
    return out


def expert_cache(cfg, seed, steps, frac=0.25, hybrid_steps=128):
    """The 3B shape with Q4_0 weights and the Zipf(1.1) router bias, experts served from an HBM pool holding 25% of
    the 1280 experts (320 slots) over pinned host memory: `steps` greedy tokens from an empty pool, one graph per
    token (routing, LRU and the host->pool copies all on the device). Reports tok/s, the hit rate, the bytes copied
    per token, the copy kernel's PCIe rate, and the same model fully resident for comparison."""
    import numpy as np

    import moert
    log("expert cache: building the 3B Q4_0 model")
    m = moert.SynthModel(cfg, seed=seed + 5, wdtype=moert.Q4_0, embed_dtype=moert.Q4_0, zipf_s=1.1)
    slots = int(cfg.layers * cfg.experts * frac)
    # the decode bench's cache shape (4416 positions, 32 requested splits: 23 splits of 3 tiles), where the
    # attention block applies and the prefetch runs inside its launch
    max_len, splits = max(4416, (steps + 2 + 63) // 64 * 64), 32
    record = moert.dtype_bytes(moert.Q4_0, 3 * cfg.inter * cfg.hidden)
    tok = int(np.random.default_rng(seed).integers(0, cfg.vocab))
    g = moert.GpuModel(m, max_len, attn_splits=splits, cache_slots=slots)
    log(f"expert cache: pinned host store and {slots}-slot pool ready; greedy run")
    g.step(tok, want_logits=False)
    g.cache_clear()
    g.reset()
    g.step(tok, want_logits=False)
    t0 = time.perf_counter()
    g.time_steps(0, steps - 1)
    wall = time.perf_counter() - t0
    hits, copies = g.cache_stats()
    n = steps * cfg.layers * cfg.top_k
    tok_s = (steps - 1) / wall
    # the same positions with a forced stream of random tokens (greedy decoding of a random-init model settles on
    # one token, and so on one set of experts per layer); one graph replay per token, no host synchronisation
    log("expert cache: forced-token run")
    forced = np.random.default_rng(seed + 1).integers(0, cfg.vocab, steps)
    g.cache_clear()
    g.reset()
    t0 = time.perf_counter()
    g.generate(forced, 1)
    fwall = time.perf_counter() - t0
    fhits, fcopies = g.cache_stats()
    # the same forced run with the prefetch: each layer's experts predicted from the layer's input (its norm and
    # router applied to the residual before attention) and copied into the pool, inside the attention launch (the
    # default where the block applies) and as the side-stream branch beside the three-kernel attention
    def prefetched_run(label, branch):
        log(f"expert cache: forced-token run with the prefetch {label}")
        if branch:
            os.environ["MOERT_PF_BLOCK"] = "0"
        try:
            g.cache_prefetch_mode(True)
        finally:
            os.environ.pop("MOERT_PF_BLOCK", None)
        path = g.kernel_path()
        g.cache_clear()
        g.reset()
        c0 = g.cache_counters()
        t0 = time.perf_counter()
        g.generate(forced, 1)
        pwall = time.perf_counter() - t0
        c1 = g.cache_counters()
        # its cost alone: the greedy run (all hits after its first steps) with the prefetch on
        g.reset()
        g.step(tok, want_logits=False)
        t0 = time.perf_counter()
        g.time_steps(0, steps - 1)
        pgreedy = (steps - 1) / (time.perf_counter() - t0)
        g.cache_prefetch_mode(False)
        pc = {k: c1[k] - c0[k] for k in ("hits", "copies", "prefetched")}
        # miss bytes overlapped: the records copied ahead, of all records copied in the run
        return {"kernel_path": path, "tok_s": round((steps + 1) / pwall, 2), "hits": pc["hits"],
                "copies_in_step": pc["copies"], "prefetched": pc["prefetched"],
                "overlapped_miss_bytes_frac": round(pc["prefetched"] / max(1, pc["prefetched"] + pc["copies"]), 4),
                "copied_bytes_per_token": round((pc["copies"] + pc["prefetched"]) * record / steps),
                "greedy_tok_s": round(pgreedy, 2)}

    prefetch = prefetched_run("inside the attention launch", False)
    prefetch["side_branch"] = prefetched_run("branch", True)
    # the greedy run without prefetch on this model again, beside the prefetched ones (same shape and box state)
    g.reset()
    g.step(tok, want_logits=False)
    t0 = time.perf_counter()
    g.time_steps(0, steps - 1)
    prefetch["greedy_tok_s_without"] = round((steps - 1) / (time.perf_counter() - t0), 2)
    # the empty pool filled from the host between steps (moert_cache_fill: each slot's record copied with
    # hipMemcpyAsync on a side stream, host-timed including the table read-back and write-back)
    g.cache_clear()
    t0 = time.perf_counter()
    filled = g.cache_fill()
    fill_s = time.perf_counter() - t0
    g.close()
    # the host-CPU hybrid on the same model and forced tokens: experts outside the token's table computed on the host
    # (16 threads), LFU admission with the reference's backlog of 4 copies, copies queued behind the layer
    hsteps = min(steps, hybrid_steps)
    hybrid = None
    if hsteps > 0:
        log(f"expert cache: host-CPU hybrid, {hsteps} forced tokens")
        hy = moert.GpuModel(m, max_len, attn_splits=splits, hybrid=(slots, 4, 16))
        t0 = time.perf_counter()
        hy.generate(forced[:hsteps], 1)
        hwall = time.perf_counter() - t0
        hc = hy.cache_counters()
        hy.close()
        hybrid = {"tok_s": round((hsteps + 1) / hwall, 2), "steps": hsteps + 1, "cpu_threads": 16, "backlog": 4,
                  **{k: hc[k] for k in ("needed", "hits", "cpu", "copies", "dropped", "deferred")},
                  "hit_frac": round(hc["hits"] / max(1, hc["needed"]), 4)}
    probe_bytes = 256 << 20
    pk, pm = moert.h2d_probe(probe_bytes, 4)
    log("expert cache: resident comparison")
    r = moert.GpuModel(m, max_len, attn_splits=splits)
    r.step(tok, want_logits=False)
    res_ms = r.time_steps(2, 64)
    r.close()
    out = {"slots": slots, "experts_total": cfg.layers * cfg.experts, "steps": steps, "max_len": max_len,
           "attn_splits": splits, "tok_s": round(tok_s, 2),
           "ms_per_step": round(wall * 1e3 / (steps - 1), 4), "hits": hits, "copies": copies,
           "hit_rate": round(hits / max(1, hits + copies), 4), "requests": n,
           "copied_bytes_per_token": round(copies * record / steps),
           "forced_tokens": {"tok_s": round((steps + 1) / fwall, 2), "hits": fhits, "copies": fcopies,
                             "hit_rate": round(fhits / max(1, fhits + fcopies), 4),
                             "copied_bytes_per_token": round(fcopies * record / steps),
                             "pcie_gbs_end_to_end": round(fcopies * record / fwall / 1e9, 2)},
           "forced_tokens_prefetch": prefetch,
           "forced_tokens_hybrid": hybrid,
           "h2d_probe": {"bytes": probe_bytes, "kernel_copy_gbs": round(probe_bytes / (pk * 1e-6) / 1e9, 2),
                         "hipmemcpy_gbs": round(probe_bytes / (pm * 1e-6) / 1e9, 2)},
           "fill": {"experts": filled, "bytes": filled * record, "ms": round(fill_s * 1e3, 2),
                    "gbs": round(filled * record / fill_s / 1e9, 2)},
           "resident_tok_s": round(1e3 / res_ms, 2)}
    log(f"expert cache {slots}/{cfg.layers * cfg.experts} slots: {tok_s:.1f} tok/s, hit rate {out['hit_rate']:.3f}, "
        f"{out['copied_bytes_per_token'] / 1e6:.1f} MB copied per token; resident {out['resident_tok_s']} tok/s; "
        f"forced tokens {out['forced_tokens']}; with prefetch {prefetch}; fill {out['fill']}")
    return out


def host_cpu():
    """The host's logical CPU count, the cores this process may run on, the per-GPU share the host sets through
    OMP_NUM_THREADS (when set), and the CPU model name."""
    nproc = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = nproc
    share = os.environ.get("OMP_NUM_THREADS", "")
    usable = min(affinity, int(share)) if share.isdigit() and int(share) > 0 else affinity
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": nproc, "affinity": affinity, "usable": usable, "model": model}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--kernel-iters", type=int, default=6)
    ap.add_argument("--cpu-steps", type=int, default=32,
                    help="decode steps of the CPU port of the reference CPU path timed for the CPU baseline")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="threads of the CPU baseline (0: every core this process may run on, within the host's "
                         "per-GPU share given by OMP_NUM_THREADS when it is set)")
    ap.add_argument("--seed", type=int, default=3003)
    ap.add_argument("--attn-splits", type=int, default=32,
                    help="KV splits requested for decode attention (tiles per split = ceil(tiles / splits))")
    ap.add_argument("--cache-steps", type=int, default=512,
                    help="greedy steps of the 3B Q4_0 model served from a 25%% expert cache (0 skips it)")
    ap.add_argument("--prefill-reps", type=int, default=5,
                    help="timed multi-position steps of 32 positions after the cached context (0: none)")
    ap.add_argument("--batched-iters", type=int, default=20,
                    help="rounds of the 16-position grouped MoE step over 4 rotating 3B blocks (0 skips it)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this engine has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np

    import moert

    n, name = moert.device_info()
    if n < 1:
        log("no GPU visible")
        sys.exit(1)
    cfg = moert.Config(**moert.GRANITE_3B)
    wd = ed = moert.Q8_0
    log(f"device {name}; building the 3B model")
    t = time.time()
    model = moert.SynthModel(cfg, seed=args.seed, wdtype=wd, embed_dtype=ed)
    log(f"weights {model.weight_bytes() / 1e9:.2f} GB in {time.time() - t:.1f} s")
    max_len = (CTX + 1 + args.warmup + args.steps + 63) // 64 * 64
    g = moert.GpuModel(model, max_len, attn_splits=args.attn_splits)
    kv = [moert.kv_prefill_data(cfg, args.seed, l, CTX) for l in range(cfg.layers)]
    for l, (k, v) in enumerate(kv):
        g.kv_prefill(l, k, v)
    log(f"uploaded; KV pre-filled to {CTX} positions")
    tok = int(np.random.default_rng(args.seed).integers(0, cfg.vocab))
    g.set_position(CTX)
    g.step(tok, want_logits=False)
    if args.warmup:
        g.time_steps(args.warmup, 0)
    pos0 = g.position()
    t0 = time.perf_counter()
    ms_event = g.time_steps(0, args.steps)
    wall = time.perf_counter() - t0
    tok_s = args.steps / wall
    ctx_mean = pos0 + (args.steps - 1) / 2.0
    step_bytes = moert.step_bytes(cfg, wd, ed, int(round(ctx_mean)))
    log(f"{args.steps} steps in {wall * 1e3:.1f} ms wall ({ms_event:.3f} ms/step by events): {tok_s:.1f} tok/s")

    kernels = {}
    nsplit = moert.attn_splits_for(max_len, moert.tiles_per_split(max_len, args.attn_splits))
    for kind in range(len(moert.KERNEL_NAMES)):
        g.set_position(pos0)
        us, launches = g.time_kernel(kind, args.kernel_iters)
        per_step = launches // args.kernel_iters
        if launches == 0:
            continue  # a class this step does not launch (the attention block replaces three of them)
        nbytes = kernel_bytes(kind, cfg, pos0 + args.kernel_iters // 2, wd, ed, nsplit)
        kernels[moert.KERNEL_NAMES[kind]] = {
            "us": round(us, 3), "launches_per_step": per_step, "bytes": nbytes,
            "gbs": round(nbytes / (us * 1e-6) / 1e9, 1) if nbytes else None, "us_per_step": round(us * per_step, 2)}
    dom = max(kernels, key=lambda k: kernels[k]["us_per_step"])
    dk = kernels[dom]
    log("kernels: " + ", ".join(f"{k} {v['us']:.2f}us x{v['launches_per_step']} {v['gbs'] or 0:.0f}GB/s"
                                for k, v in kernels.items()))
    # the MoE GEMV of the metric: its own kernels, or (one launch per layer) inside the layer kernel
    moe = {k: kernels[k] for k in ("route_up", "expert_down", "moe_xcd", "layer") if k in kernels}
    prefill = prefill_block(g, cfg, args.seed, CTX, tok_s, reps=args.prefill_reps) if args.prefill_reps > 0 else None
    g.close()
    copy_bytes = 1 << 30
    copy_us = moert.copy_probe(copy_bytes, 10)
    hbm_copy = {"bytes_moved": 2 * copy_bytes, "us": round(copy_us, 2),
                "gbs": round(2 * copy_bytes / (copy_us * 1e-6) / 1e9, 1)}
    log(f"device copy of {copy_bytes >> 20} MiB: {copy_us:.1f} us, {hbm_copy['gbs']:.0f} GB/s read+write")
    # cold streaming reads: the achievable read rate of a long stream, and of one of the size of a grouped gate/up
    # launch at 16 positions (40 MiB), which includes the ramp-up every launch pays
    hbm_read = []
    for rb in (1 << 30, 40 << 20):
        r_us = moert.read_probe(rb, 10)
        hbm_read.append({"bytes": rb, "us": round(r_us, 2), "gbs": round(rb / (r_us * 1e-6) / 1e9, 1)})
        log(f"cold read of {rb >> 20} MiB: {r_us:.1f} us, {hbm_read[-1]['gbs']:.0f} GB/s")

    batched = batched_step(cfg, args.seed, args.batched_iters) if args.batched_iters > 0 else None
    cache = expert_cache(cfg, args.seed, args.cache_steps) if args.cache_steps > 0 else None

    cpu = None
    if args.cpu_steps > 0:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle
        hw = host_cpu()
        threads = args.cpu_threads or hw["usable"]
        s = oracle.PortSession(model, max_len, threads=threads)
        for l, (k, v) in enumerate(kv):
            s.kv_prefill(l, k, v)
        s.set_position(CTX)
        s.step(tok)
        t0 = time.perf_counter()
        nxt = tok
        for _ in range(args.cpu_steps):
            lg = s.step(nxt)[0]
            nxt = oracle.argmax(lg)
        cw = time.perf_counter() - t0
        cpu = {"value": round(args.cpu_steps / cw, 3), "unit": "tok/s", "cores": threads, "kind": "port",
               "nproc": hw["nproc"], "affinity": hw["affinity"], "cpu_model": hw["model"],
               "sample": f"{args.cpu_steps} greedy decode steps of the same 3B Q8_0 model at context {CTX + 1}.."
                         f"{CTX + args.cpu_steps}: C++ port of the reference CPU path (CpuSession::step, dot_avx2's "
                         f"4x8-lane accumulation on Q8_0 blocks, 16-row pool tasks, f32 KV, attention on the "
                         f"calling thread), {threads} threads ({cw:.1f} s)"}
        log(f"cpu baseline {cpu['value']} tok/s on {threads} threads of {hw['model']} (nproc {hw['nproc']})")

    out = {
        "metric": "decode tok/s batch1 (3B-A800M shape); MoE GEMV achieved HBM GB/s vs peak",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "granite-3b-a800m greedy decode, batch 1, q8_0 weights and tied head, fp16 kv "
                               f"pre-filled to {CTX}", "layers": cfg.layers, "hidden": cfg.hidden,
                   "experts": cfg.experts, "top_k": cfg.top_k, "context_mean": ctx_mean, "parallelism": "none"},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": dk["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dk["gbs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom),
                     "algorithmic_bytes": dk["bytes"], "us": dk["us"],
                     "traffic_source": "profiles/decode3b_hbm_traffic.md (FETCH_SIZE x2 + WRITE_SIZE, k_copy-calibrated)"},
        "step_roofline": {"bytes": step_bytes, "achieved": round(step_bytes / (wall / args.steps) / 1e9, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(step_bytes / (wall / args.steps) / 1e9 / HBM_PEAK_GBS, 4)},
        "moe_gemv": moe,
        "hbm_copy": hbm_copy,
        "hbm_read": hbm_read,
        "batched_step": batched,
        "prefill_block": prefill,
        "expert_cache": cache,
        "kernels": kernels,
        "cpu_baseline": cpu,
        "device": name,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
