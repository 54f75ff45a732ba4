#!/usr/bin/env python3
"""Stories110M fp16 batch-1 greedy decode throughput on one MI355X.

One step = one full greedy Decode (ane/stories/infer.go:136-202) of the synthetic workload:
Stories110M shape (12 layers, dim 768, 12 heads, SwiGLU 2048, vocab 32000), N(0, 0.02)
weights from seed 0 stored as fp16 and resident in HBM, a 16-id prompt from seed 1, 128 new
tokens (143 token forwards). `value` is generated tokens per second of wall time over the
timed steps, as cmd/stories-generate-go/main.go:54-58 counts them.

The JSON line also carries:
  roofline      the per-token forward (the dominant work): algorithmic bytes per forward
                divided by its device time from HIP events on the library's stream,
                against the 8 TB/s HBM peak;
  cpu_baseline  the CPU restatement of infer.go (oracle/, test infrastructure) timed on
                one host core over the same decode, with its token stream compared.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ane-training-experiments_amd"))

METRIC = "batch-1 decode tokens/sec (Stories110M, Qwen3-0.6B); achieved HBM GB/s"
HBM_PEAK_GBS = 8000.0
PROMPT_LEN, NEW_TOKENS = 16, 128


def cpu_baseline(cfg, weights, prompt, gpu_tokens):
    """The oracle's decode (a port of infer.go) on 1 thread over the full workload."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    import stories_hip as sh

    dec = oracle.Decoder(oracle.config_from(cfg), weights.rounded(sh.SH_DTYPE_F16), threads=1)
    t0 = time.perf_counter()
    toks, _, _ = dec.greedy_decode(prompt, NEW_TOKENS)
    dt = time.perf_counter() - t0
    gen = len(toks) - len(prompt)
    return {
        "value": round(gen / dt, 3),
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": f"full workload: {len(prompt)}-id prompt + {gen} new tokens "
                  f"({len(prompt) - 1 + gen} forwards), C restatement of infer.go, 1 thread, "
                  f"{dt:.2f} s",
        "tokens_match_gpu": toks.tolist() == gpu_tokens,
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "this build has no multi-GPU path", file=sys.stderr)
        return 2

    import stories_hip as sh

    sh.init(0)
    cfg = sh.stories110m_config()
    weights = sh.synth_weights(cfg, seed=0, std=0.02)
    model = sh.Model(cfg, sh.SH_DTYPE_F16)
    model.upload(weights)
    prompt = sh.synth_tokens(PROMPT_LEN, 1, cfg.vocab)

    for _ in range(args.warmup):
        model.greedy_decode(prompt, NEW_TOKENS)

    gen_tokens = 0
    forwards = 0
    gpu_ms = 0.0
    bytes_total = 0.0
    toks = None
    t0 = time.perf_counter()
    for _ in range(args.steps):
        toks, plen, _ = model.greedy_decode(prompt, NEW_TOKENS)  # synchronous
        st = model.stats()
        gen_tokens += len(toks) - plen
        forwards += st["forwards"]
        gpu_ms += st["gpu_ms"]
        bytes_total += st["bytes_per_forward_mean"] * st["forwards"]
    wall = time.perf_counter() - t0

    fwd_us = gpu_ms * 1e3 / max(forwards, 1)
    achieved = bytes_total / (gpu_ms / 1e3) / 1e9 if gpu_ms > 0 else 0.0
    line = {
        "metric": METRIC,
        "value": round(gen_tokens / wall, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: N(0,0.02) weights seed 0 (fp16), 16-id prompt seed 1",
        "config": {
            "workload": "Stories110M fp16 batch-1 greedy decode, 16-id prompt + 128 new tokens",
            "layers": cfg.n_layers, "dim": cfg.dim, "heads": cfg.n_heads, "hidden": cfg.hidden,
            "vocab": cfg.vocab, "batch": 1, "prompt_tokens": PROMPT_LEN, "new_tokens": NEW_TOKENS,
            "kv_cache": "fp32", "parallelism": "none (1 GPU)",
        },
        "roofline": {
            "kernel": ("k_decode_persistent (whole decode in one launch; per-forward figures)"
                       if st["persistent"] else "token forward (all kernels of one position)"),
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "bytes_per_forward": round(bytes_total / max(forwards, 1)),
            "us_per_forward": round(fwd_us, 3),
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, weights, prompt, toks.tolist())
    model.close()
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
