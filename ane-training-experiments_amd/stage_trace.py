#!/usr/bin/env python3
"""Stage trace of the persistent decode kernel: where one token forward's time goes.

A tracing aid like the reference's per-step buckets (ane/storiesane/metrics.go:13-60). It runs
a greedy decode of a synthetic model twice (the first warms the model up), arms
sh_trace_forward for one forward of the second, and reads the per-workgroup constant-clock
stamps back (sh_trace_read): for every stage the time each workgroup had its whole input
(input ready) and the time it had issued its output stores (end). For each stage of each
layer it reports, on the critical path,

  hand-over  from the previous stage's last end stamp to this stage's last input-ready stamp
             (the producers' store latency, the consumers' detection of the last word and
             their input staging: the cost of one grid-wide exchange);
  in-stage   from that input-ready stamp to this stage's last end stamp (the arithmetic, the
             output staging and the store issue).

Usage:
  python stage_trace.py [--shape stories110m|qwen3-0.6b] [--dtype fp16|bf16|w8a8]
                        [--prompt-len 16] [--max-new 128] [--forward 85] [--json FILE]
"""
import argparse
import json
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import stories_hip as sh  # noqa: E402

STAGES = ["qkv", "attn", "wo", "w13", "w2"]


def trace(shape="stories110m", dtype="fp16", prompt_len=16, max_new=128, forward=85, seed=None):
    cfg = sh.stories110m_config() if shape == "stories110m" else sh.qwen3_06b_config()
    dt = {"fp16": sh.SH_DTYPE_F16, "bf16": sh.SH_DTYPE_BF16, "w8a8": sh.SH_DTYPE_W8A8}[dtype]
    wseed = seed if seed is not None else (0 if shape == "stories110m" else 3)
    w = sh.synth_weights(cfg, seed=wseed, std=0.02)
    m = sh.Model(cfg, dt)
    m.upload(w)
    del w
    prompt = sh.synth_tokens(prompt_len, 1 if shape == "stories110m" else 3, cfg.vocab)
    m.greedy_decode(prompt, max_new)
    m.trace_forward(forward)
    m.greedy_decode(prompt, max_new)
    st = m.stats()
    E, I = m.trace_stamps(), m.trace_inputs()
    L = cfg.n_layers
    rows = []
    for l in range(L):
        for j, name in enumerate(STAGES):
            c = 1 + 5 * l + j
            prev_end = float(np.nanmax(E[:, c - 1]))
            has = ~np.isnan(I[:, c])
            ready = float(np.nanmax(I[has, c]))
            end = float(np.nanmax(E[has, c]))
            rows.append({"layer": l, "stage": name, "hand_over_us": ready - prev_end, "in_stage_us": end - ready,
                         "consumers": int(has.sum())})
    for k, name in enumerate(["classifier", "argmax"]):
        c = 1 + 5 * L + k
        prev_end = float(np.nanmax(E[:, c - 1]))
        ready = float(np.nanmax(I[:, c]))
        end = float(np.nanmax(E[:, c]))
        rows.append({"layer": None, "stage": name, "hand_over_us": ready - prev_end, "in_stage_us": end - ready,
                     "consumers": int((~np.isnan(I[:, c])).sum())})
    out = {
        "shape": shape, "dtype": dtype, "prompt_len": prompt_len, "max_new": max_new, "forward": forward,
        "position": prompt_len - 1 + forward, "describe": m.describe(),
        "launch_us_per_forward": 1000.0 * (st["gpu_ms"] - st["prefill_ms"]) / st["forwards"],
        "traced_forward_us": float(np.nanmax(E[:, -1]) - np.nanmin(E[:, 0])),
        "rows": rows,
    }
    m.close()
    return out


def markdown(t):
    lines = [f"Traced forward {t['forward']} (position {t['position']}) of a {t['prompt_len']}-id prompt + "
             f"{t['max_new']}-token greedy decode, {t['shape']} {t['dtype']}: "
             f"{t['traced_forward_us']:.1f} µs (launch mean {t['launch_us_per_forward']:.1f} µs per forward).", "",
             "Per stage, summed over the layers (µs):", "",
             "| stage | hand-over | in-stage | total | consumers |", "|---|---:|---:|---:|---:|"]
    tot_h = tot_w = 0.0
    for name in STAGES + ["classifier", "argmax"]:
        rs = [r for r in t["rows"] if r["stage"] == name]
        h = sum(r["hand_over_us"] for r in rs)
        w = sum(r["in_stage_us"] for r in rs)
        tot_h += h
        tot_w += w
        lines.append(f"| {name} | {h:.1f} | {w:.1f} | {h + w:.1f} | {rs[0]['consumers']} |")
    lines.append(f"| all | {tot_h:.1f} | {tot_w:.1f} | {tot_h + tot_w:.1f} | |")
    lines += ["", "One layer (µs): hand-over / in-stage per stage.", "",
              "| layer | " + " | ".join(STAGES) + " |", "|---|" + "---:|" * len(STAGES)]
    layers = sorted({r["layer"] for r in t["rows"] if r["layer"] is not None})
    for l in (layers[0], layers[len(layers) // 2], layers[-1]):
        rs = {r["stage"]: r for r in t["rows"] if r["layer"] == l}
        lines.append(f"| {l} | " + " | ".join(f"{rs[s]['hand_over_us']:.2f} / {rs[s]['in_stage_us']:.2f}"
                                           for s in STAGES) + " |")
    return "\n".join(lines)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--shape", default="stories110m", choices=["stories110m", "qwen3-0.6b"])
    ap.add_argument("--dtype", default=None, choices=["fp16", "bf16", "w8a8"])
    ap.add_argument("--prompt-len", type=int, default=None)
    ap.add_argument("--max-new", type=int, default=None)
    ap.add_argument("--forward", type=int, default=85)
    ap.add_argument("--json", default=None)
    a = ap.parse_args()
    qwen = a.shape == "qwen3-0.6b"
    t = trace(a.shape, a.dtype or ("bf16" if qwen else "fp16"), a.prompt_len or (32 if qwen else 16),
              a.max_new or (256 if qwen else 128), a.forward)
    print(markdown(t))
    if a.json:
        with open(a.json, "w") as f:
            json.dump(t, f, indent=1)


if __name__ == "__main__":
    main()
