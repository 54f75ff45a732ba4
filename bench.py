#!/usr/bin/env python3
"""Stories110M fp16 batch-1 greedy decode throughput on one MI355X.

One step = one full greedy Decode (ane/stories/infer.go:136-202) of the synthetic workload:
Stories110M shape (12 layers, dim 768, 12 heads, SwiGLU 2048, vocab 32000), N(0, 0.02)
weights from seed 0 stored as fp16 and resident in HBM, a 16-id prompt from seed 1, 128 new
tokens (143 token forwards). `value` is generated tokens per second of wall time over the
timed steps, as cmd/stories-generate-go/main.go:54-58 counts them.

The GPU leg runs in the C++ host program (ane-training-experiments_amd/stories-generate
-bench-steps K -bench-warmup W), a child process; it times the K steps with a steady clock
around the whole decode calls and reads each call's device time from HIP events on the
library's stream (sh_stats). This process touches no GPU.

The JSON line also carries:
  roofline      the dominant kernel, k_decode_persistent (one launch runs a whole decode):
                algorithmic bytes per launch (the sum over its token forwards of weights,
                norms, KV rows read and written, logits) divided by the launch's device time,
                against the 8 TB/s HBM peak. `traffic` is the HBM bytes per launch from the
                profiler's FETCH_SIZE and WRITE_SIZE counters, each scaled by what the same
                counter reads over a plain copy kernel of known size (figures kept in
                profiles/, null when absent); `copy_gbs` is that copy kernel's bandwidth
                measured in this run;
  cpu_baseline  the CPU restatement of infer.go (oracle/, test infrastructure) timed on
                one host core over the same decode, with its token stream compared.
"""
import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "ane-training-experiments_amd")
CLI = os.path.join(PKG, "stories-generate")
sys.path.insert(0, PKG)

METRIC = "batch-1 decode tokens/sec (Stories110M, Qwen3-0.6B); achieved HBM GB/s"
HBM_PEAK_GBS = 8000.0
PROMPT_LEN, NEW_TOKENS = 16, 128
COPY_BYTES = 1 << 30
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k_decode_persistent_stories110m_traffic.json")


def traffic_per_launch():
    """HBM bytes per k_decode_persistent launch from the committed counter figures: each
    counter's KiB per dispatch times (known copy bytes / the counter's KiB over the copy)."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        fetch = t["kernel"]["FETCH_SIZE_kib"] * t["copy"]["bytes_read"] / t["copy"]["FETCH_SIZE_kib"]
        write = t["kernel"]["WRITE_SIZE_kib"] * t["copy"]["bytes_written"] / t["copy"]["WRITE_SIZE_kib"]
        return round(fetch + write)
    except (OSError, KeyError, ValueError, ZeroDivisionError):
        return None


def gpu_leg(steps, warmup):
    """Runs the timed decodes in the host program and returns its JSON result."""
    if not os.path.exists(CLI):
        raise SystemExit(f"{CLI} is not built: run `make -C {PKG}` (or __graft_entry__.build())")
    cmd = [CLI, "-shape", "stories110m", "-dtype", "fp16", "-synthetic-seed", "0",
           "-synthetic-std", "0.02", "-prompt-len", str(PROMPT_LEN), "-prompt-seed", "1",
           "-max-new", str(NEW_TOKENS), "-bench-steps", str(steps), "-bench-warmup", str(warmup),
           "-copy-calibrate", str(COPY_BYTES)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    sys.stderr.write(p.stderr)
    result = None
    for line in p.stdout.splitlines():
        if line.startswith("{"):
            result = json.loads(line)
    if p.returncode != 0:
        # rocprofv3 can end a program that launched a cooperative kernel with SIGSEGV in its
        # own teardown, after the program printed its result; only then is the result kept.
        profiled = any(k.startswith("ROCPROF") for k in os.environ)
        if not (profiled and result is not None and p.returncode == -11):
            raise SystemExit(f"stories-generate failed (exit {p.returncode})")
        print("note: stories-generate ended with signal 11 after printing its result "
              "(profiler teardown)", file=sys.stderr)
    if result is None:
        raise SystemExit("stories-generate printed no result")
    return result


def cpu_baseline(gpu_tokens):
    """The oracle's decode (a port of infer.go) on 1 thread over the full workload."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    import stories_hip as sh

    cfg = sh.stories110m_config()
    weights = sh.synth_weights(cfg, seed=0, std=0.02)
    prompt = sh.synth_tokens(PROMPT_LEN, 1, cfg.vocab)
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

    r = gpu_leg(args.steps, args.warmup)
    steps = r["steps"]
    gen_tokens = sum(r["generated"])
    forwards = sum(r["forwards"])
    gpu_ms = sum(r["gpu_ms"])
    bytes_total = sum(b * f for b, f in zip(r["bytes_per_forward_mean"], r["forwards"]))
    wall = r["wall_s"]
    launch_ms = gpu_ms / steps
    bytes_launch = bytes_total / steps
    achieved = bytes_launch / (launch_ms / 1e3) / 1e9 if gpu_ms > 0 else 0.0
    persistent = bool(r["persistent"])
    line = {
        "metric": METRIC,
        "value": round(gen_tokens / wall, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": r["warmup"],
        "ms_per_step": round(wall * 1e3 / steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: N(0,0.02) weights seed 0 (fp16), 16-id prompt seed 1",
        "config": {
            "workload": "Stories110M fp16 batch-1 greedy decode, 16-id prompt + 128 new tokens",
            "layers": 12, "dim": 768, "heads": 12, "hidden": 2048, "vocab": 32000, "batch": 1,
            "prompt_tokens": PROMPT_LEN, "new_tokens": NEW_TOKENS, "kv_cache": "fp32",
            "parallelism": "none (1 GPU)",
        },
        "roofline": {
            "kernel": ("k_decode_persistent (one launch = one whole decode)" if persistent
                       else "per-stage decode kernels (all launches of one decode)"),
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_per_launch() if persistent else None,
            "bytes_per_launch": round(bytes_launch),
            "launch_ms": round(launch_ms, 4),
            "forwards_per_launch": forwards // steps,
            "us_per_forward": round(gpu_ms * 1e3 / max(forwards, 1), 3),
            "copy_gbs": round(r["copy_gbs"], 1),
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(r["tokens"])
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
