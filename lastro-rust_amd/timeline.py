#!/usr/bin/env python3
"""Per-workgroup phase timeline of the batch-1 decode step (measurement build libmoert_tl.so).

Builds the decode workload of bench.py (Granite-3B-A800M shape, Q8_0 weights and tied head, fp16 KV pre-filled with
N(0, 1) to 4096 positions, 32 KV splits requested), replays the step graph with every workgroup of every launch
stamping the 100 MHz real-time clock at its phase boundaries, and prints a markdown summary per kernel class:

  span        first workgroup start to last workgroup end of a launch
  gap before  end of the previous launch (its last workgroup) to this launch's first workgroup start
  start ramp  first to last workgroup start of a launch (dispatch of the grid)
  wave skew   first to last wave start inside a workgroup
  life        a workgroup's first wave start to its last wave end
  phases      time from a workgroup's first wave start to the end of each phase, as its wave 0 sees it
  latest      time from a launch's first workgroup start to the end of each phase in its latest workgroup

All figures are medians over the workgroups (or launches) of --steps steps after --warmup untimed ones.
Usage: python lastro-rust_amd/timeline.py [--steps 8] [--out FILE]
"""
import argparse
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import moert  # noqa: E402

TICK_US = 0.01  # s_memrealtime runs at 100 MHz
END = moert.TL_WORDS - 1  # word of the latest wave end
NPH = moert.TL_WORDS - 3  # phase-end words 2 .. END - 1
PHASES = {
    "embed": [],
    "qkv": ["norm of h (staged, sum of squares)", "q/k/v rows fma"],
    "attn_split": ["K tiles in LDS", "scores + tile maxima", "p, V tiles in LDS", "p.v"],
    "attn_combine": ["partials loaded, max"],
    "oproj": ["att staged", "o rows fma"],
    "route_up": ["norm of h", "router logits in LDS", "rank + ids", "expert gate/up rows fma"],
    "expert_down": ["activations staged", "down rows fma"],
    "head": ["norm of h"],
    "head_argmax": [],
    "attn_block": ["q/k/v rows fma", "tiles staged", "queries in", "partials stored", "merge done"],
    "moe_xcd": ["norm of h, router logits in LDS", "rank + ids", "gate/up rows fma", "act of the XCD's expert in"],
    "moe_combine": [],
    "layer": ["input + norm", "partials / merge done", "merged heads in", "o rows done", "h' gathered",
              "router items out", "logits in", "ranked", "act of the XCD's expert in"],
    "layer_combine": [],
}


def summarize(records, kinds):
    """records: list over steps of (rec [launches, 1024, moert.TL_WORDS] u64, kinds [launches])."""
    rows = {}
    totals = []
    for rec, kd in records:
        starts, ends = [], []
        for i in range(len(kd)):
            r = rec[i]
            used = r[:, END] != 0
            r = r[used].astype(np.int64)
            first = (~rec[i][used][:, 0]).astype(np.int64)
            last_start, end = r[:, 1], r[:, END]
            starts.append(first.min())
            ends.append(end.max())
            name = moert.KERNEL_NAMES[kd[i]]
            d = rows.setdefault(name, {"span": [], "gap": [], "ramp": [], "skew": [], "life": [], "blocks": [],
                                       "phases": [[] for _ in range(NPH)], "last": [[] for _ in range(NPH)]})
            d["span"].append(end.max() - first.min())
            d["ramp"].append(first.max() - first.min())
            d["skew"].extend((last_start - first).tolist())
            d["life"].extend((end - first).tolist())
            d["blocks"].append(int(used.sum()))
            for ph in range(NPH):
                col = r[:, 2 + ph]
                ok = col != 0
                if ok.any():
                    d["phases"][ph].extend((col[ok] - first[ok]).tolist())
                    d["last"][ph].append(int(col[ok].max() - first.min()))
            if i > 0:
                d["gap"].append(starts[-1] - ends[-2])
        totals.append(ends[-1] - starts[0])
    return rows, totals


def med(v):
    return float(np.median(v)) * TICK_US if len(v) else float("nan")


def render(rows, totals, steps, launches):
    out = []
    out.append(f"Step (first workgroup start to last workgroup end): median {med(totals):.1f} us over {steps} steps; "
               f"{launches} launches per step.\n")
    out.append("| kernel | launches/step | workgroups | span us | gap before us | start ramp us | wave skew us | "
               "life us | phase ends (us from workgroup start) | latest phase ends (us from launch start) |")
    out.append("|---|---|---|---|---|---|---|---|---|---|")
    order = [k for k in moert.KERNEL_NAMES if k in rows]
    per_step = {}
    for name in order:
        d = rows[name]
        n = len(d["span"]) // steps
        per_step[name] = n
        ph = "; ".join(f"{lab} {med(d['phases'][i]):.2f}" for i, lab in enumerate(PHASES.get(name, []))
                       if d["phases"][i])
        last = "; ".join(f"{med(d['last'][i]):.2f}" for i, _ in enumerate(PHASES.get(name, [])) if d["last"][i])
        out.append(f"| {name} | {n} | {int(np.median(d['blocks']))} | {med(d['span']):.2f} | {med(d['gap']):.2f} | "
                   f"{med(d['ramp']):.2f} | {med(d['skew']):.2f} | {med(d['life']):.2f} | {ph} | {last} |")
    span_sum = sum(med(rows[k]["span"]) * per_step[k] for k in order)
    gap_sum = sum(med(rows[k]["gap"]) * per_step[k] for k in order if rows[k]["gap"])
    out.append("")
    out.append(f"Sum of median spans x launches: {span_sum:.1f} us; sum of median gaps x launches: {gap_sum:.1f} us.")
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=8)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--seed", type=int, default=3003)
    ap.add_argument("--attn-splits", type=int, default=32)
    ap.add_argument("--out", default=None)
    ap.add_argument("--raw", default=None, help="also save the records of the first 256 workgroups (.npz)")
    args = ap.parse_args()
    moert.LIB_PATH = moert.TIMELINE_LIB_PATH
    n, name = moert.device_info()
    if n < 1:
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)
    cfg = moert.Config(**moert.GRANITE_3B)
    print("[timeline] building the 3B model", file=sys.stderr, flush=True)
    model = moert.SynthModel(cfg, seed=args.seed, wdtype=moert.Q8_0, embed_dtype=moert.Q8_0)
    ctx = 4096
    max_len = (ctx + 1 + args.warmup + args.steps + 63) // 64 * 64
    g = moert.GpuModel(model, max_len, attn_splits=args.attn_splits)
    for l in range(cfg.layers):
        k, v = moert.kv_prefill_data(cfg, args.seed, l, ctx)
        g.kv_prefill(l, k, v)
    g.set_position(ctx)
    tok = int(np.random.default_rng(args.seed).integers(0, cfg.vocab))
    g.step(tok, want_logits=False)
    print("[timeline] warm-up", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        g.timeline_step()
    records = []
    t0 = time.time()
    for i in range(args.steps):
        rec, kinds, _ = g.timeline_step()
        records.append((rec, kinds))
    print(f"[timeline] {args.steps} steps recorded in {time.time() - t0:.1f} s", file=sys.stderr, flush=True)
    rows, totals = summarize(records, None)
    text = (f"Device: {name}. Workload: 3B-A800M shape, Q8_0, fp16 KV at {ctx}..{ctx + args.warmup + args.steps}, "
            f"{args.attn_splits} KV splits requested.\n\n" + render(rows, totals, args.steps, len(records[0][1])))
    print(text)
    if args.raw:
        np.savez_compressed(args.raw, rec=np.stack([r[:, :256] for r, _ in records]), kinds=records[0][1])
    if args.out:
        with open(args.out, "w") as f:
            f.write(text + "\n")
    g.close()


if __name__ == "__main__":
    main()
