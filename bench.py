#!/usr/bin/env python3
"""Stories110M fp16 batch-1 greedy decode throughput on one MI355X.

One step = one full greedy Decode (ane/stories/infer.go:136-202) of the synthetic workload:
Stories110M shape (12 layers, dim 768, 12 heads, SwiGLU 2048, vocab 32000), N(0, 0.02)
weights from seed 0 stored as fp16 and resident in HBM, a 16-id prompt from seed 1, 128 new
tokens: the prompt's first 15 positions fill the KV cache in one full-sequence forward, then
one k_decode_persistent launch runs the 128 token forwards. `value` is generated tokens per
second of wall time over the timed steps, as cmd/stories-generate-go/main.go:54-58 counts
them.

The GPU leg runs in the C++ host program (ane-training-experiments_amd/stories-generate
-bench-steps K -bench-warmup W), a child process; it times the K steps with a steady clock
around the whole decode calls and reads each call's device time from HIP events on the
library's stream (sh_stats). This process touches no GPU.

The JSON line also carries:
  roofline      the dominant kernel, k_decode_persistent (one launch runs a whole decode):
                algorithmic bytes per launch (the sum over its token forwards of weights,
                norms, KV rows read and written, logits) divided by the launch's device time
                (each decode's HIP-event time less its prompt forward, reported as
                prompt_forward_ms), against the 8 TB/s HBM peak. `traffic` is the HBM bytes
                per launch from the
                profiler's FETCH_SIZE and WRITE_SIZE counters, each scaled by what the same
                counter reads over a plain copy kernel of known size (figures kept in
                profiles/, null when absent); `copy_gbs` is that copy kernel's bandwidth
                measured in this run, `read_gbs` a read-only stream's (the practical
                ceiling for a path whose traffic is almost all reads);
  cpu_baseline  the CPU restatement of infer.go (oracle/, test infrastructure) timed on
                one host core over the same decode, with its token stream compared.

`--workload` selects one of the other measured configurations instead (same JSON contract,
each with its own roofline and a bounded CPU sample):
  prefill      Stories110M EvalLogits forward, S = 256 (ids seed 2), α = 1/sqrt(24): MFMA-bound;
               achieved = forward FLOPs / device time; CPU: the oracle's channel-first forward
               on up to 16 host threads (the reference's GOMAXPROCS-parallel path).
  w8a8         Stories110M W8A8 greedy decode, 16-id prompt + 128 new: HBM-bound; CPU: the
               oracle's W8A8 decoder on one core.
  qwen-decode  Qwen3-0.6B-shaped bf16 greedy decode, 32-id prompt (seed 3) + 256 new:
               HBM-bound; CPU: the oracle decoder on one core over a prefix of the same decode.
  batch        Qwen3-0.6B-shaped, 32 sequences x (1024-id prompt, seed 4) + 128 greedy steps:
               HBM/KV-bound; value = generated tokens per second of the decode steps;
               CPU: the oracle decoder on one core over a short prefix of sequence 0.
  train        Stories110M training Step (storiesane Engine.Step), S = 256, fp32, over drand48
               windows of a synthetic stream: MFMA-bound (fp32 peak); value = trained tokens
               per second; CPU: the oracle's step on up to 16 host threads.
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
TRAFFIC_W8A8 = os.path.join(ROOT, "profiles", "k_decode_persistent_w8a8_stories110m_traffic.json")
TRAFFIC_QWEN = os.path.join(ROOT, "profiles", "k_decode_persistent_qwen3_traffic.json")


def traffic_per_launch(path=TRAFFIC_FILE):
    """HBM bytes per k_decode_persistent launch from the committed counter figures: each
    counter's value per dispatch times (known copy bytes / the counter's value over the copy)."""
    try:
        with open(path) as f:
            t = json.load(f)
        fetch = t["kernel"]["FETCH_SIZE_kib"] * t["copy"]["bytes_read"] / t["copy"]["FETCH_SIZE_kib"]
        write = t["kernel"]["WRITE_SIZE_kib"] * t["copy"]["bytes_written"] / t["copy"]["WRITE_SIZE_kib"]
        return round(fetch + write)
    except (OSError, KeyError, ValueError, ZeroDivisionError):
        return None


def run_cli(args):
    """Runs the host program with `args` and returns its JSON result."""
    if not os.path.exists(CLI):
        raise SystemExit(f"{CLI} is not built: run `make -C {PKG}` (or __graft_entry__.build())")
    p = subprocess.run([CLI] + [str(a) for a in args], capture_output=True, text=True)
    sys.stderr.write(p.stderr)
    result = None
    for line in p.stdout.splitlines():
        if line.startswith("{"):
            result = json.loads(line)
    if p.returncode != 0:
        raise SystemExit(f"stories-generate failed (exit {p.returncode})")
    if result is None:
        raise SystemExit("stories-generate printed no result")
    return result


def gpu_leg(steps, warmup):
    """Runs the timed decodes in the host program and returns its JSON result."""
    return run_cli(["-shape", "stories110m", "-dtype", "fp16", "-synthetic-seed", "0",
                    "-synthetic-std", "0.02", "-prompt-len", PROMPT_LEN, "-prompt-seed", "1",
                    "-max-new", NEW_TOKENS, "-bench-steps", steps, "-bench-warmup", warmup,
                    "-copy-calibrate", COPY_BYTES, "-read-calibrate", COPY_BYTES])


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


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), reported beside the CPU baseline."""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def with_host(line):
    """Adds the host description to a line's cpu_baseline: CPU model and logical cores."""
    cb = line.get("cpu_baseline")
    if isinstance(cb, dict):
        cb["cpu_model"] = cpu_model()
        cb["host_logical_cores"] = os.cpu_count()
    return line


def host_threads():
    return max(1, min(16, os.cpu_count() or 1))


def decode_line(r, steps, metric, workload, dtype, data, config, cpu, traffic_file=None):
    """JSON line of a greedy-decode workload measured by the host program's -bench-steps."""
    gen_tokens = sum(r["generated"])
    forwards = sum(r["forwards"])
    # device time of each decode = the prompt's cache-filling forward (full-sequence kernels)
    # + the token loop (one k_decode_persistent launch); the roofline is the launch's
    prefill_ms = sum(r.get("prefill_ms", [0.0] * steps))
    gpu_ms = sum(r["gpu_ms"]) - prefill_ms
    bytes_total = sum(b * f for b, f in zip(r["bytes_per_forward_mean"], r["forwards"]))
    wall = r["wall_s"]
    launch_ms = gpu_ms / steps
    bytes_launch = bytes_total / steps
    achieved = bytes_launch / (launch_ms / 1e3) / 1e9 if gpu_ms > 0 else 0.0
    persistent = bool(r["persistent"])
    line = {
        "metric": metric, "value": round(gen_tokens / wall, 2), "unit": "tokens/s", "n_gpus": 1,
        "steps": steps, "warmup": r["warmup"], "ms_per_step": round(wall * 1e3 / steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
        "data": data, "config": dict(workload=workload, **config),
        "roofline": {
            "kernel": ("k_decode_persistent (one launch = one whole decode)" if persistent
                       else "per-stage decode kernels (all launches of one decode)"),
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_per_launch(traffic_file) if persistent and traffic_file else None,
            "bytes_per_launch": round(bytes_launch), "launch_ms": round(launch_ms, 4),
            "forwards_per_launch": forwards // steps,
            "us_per_forward": round(gpu_ms * 1e3 / max(forwards, 1), 3),
            "prompt_forward_ms": round(prefill_ms / steps, 4),
        },
    }
    if cpu is not None:
        line["cpu_baseline"] = cpu(r["tokens"])
    return line


def workload_w8a8(args):
    r = run_cli(["-shape", "stories110m", "-dtype", "w8a8", "-synthetic-seed", "0",
                 "-synthetic-std", "0.02", "-prompt-len", PROMPT_LEN, "-prompt-seed", "1",
                 "-max-new", NEW_TOKENS, "-bench-steps", args.steps, "-bench-warmup", args.warmup])

    def cpu(gpu_tokens):
        import oracle
        import stories_hip as sh
        cfg = sh.stories110m_config()
        w = sh.synth_weights(cfg, seed=0, std=0.02)
        prompt = sh.synth_tokens(PROMPT_LEN, 1, cfg.vocab)
        dec = oracle.Decoder(oracle.config_from(cfg, w8a8=True), w.rounded(sh.SH_DTYPE_W8A8), threads=1)
        t0 = time.perf_counter()
        toks, _, _ = dec.greedy_decode(prompt, NEW_TOKENS)
        dt = time.perf_counter() - t0
        gen = len(toks) - len(prompt)
        return {"value": round(gen / dt, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
                "sample": f"full workload: {len(prompt)}-id prompt + {gen} new tokens, C restatement of "
                          f"infer.go with the W8A8 matVec, 1 thread, {dt:.2f} s",
                "tokens_match_gpu": toks.tolist() == gpu_tokens}

    return decode_line(r, args.steps, "batch-1 W8A8 decode tokens/sec (Stories110M)",
                       "Stories110M W8A8 batch-1 greedy decode, 16-id prompt + 128 new tokens", "int8",
                       "synthetic: N(0,0.02) weights seed 0, per-row int8 + fp32 scales, 16-id prompt seed 1",
                       {"layers": 12, "dim": 768, "vocab": 32000, "batch": 1, "prompt_tokens": PROMPT_LEN,
                        "new_tokens": NEW_TOKENS, "kv_cache": "fp32", "parallelism": "none (1 GPU)"},
                       None if args.no_cpu_baseline else cpu, TRAFFIC_W8A8)


QWEN_PROMPT, QWEN_NEW, QWEN_CPU_NEW = 32, 256, 4


def workload_qwen_decode(args):
    r = run_cli(["-shape", "qwen3-0.6b", "-dtype", "bf16", "-synthetic-seed", "3",
                 "-synthetic-std", "0.02", "-seq", QWEN_PROMPT + QWEN_NEW, "-prompt-len", QWEN_PROMPT,
                 "-prompt-seed", "3", "-max-new", QWEN_NEW, "-bench-steps", args.steps,
                 "-bench-warmup", args.warmup])

    def cpu(gpu_tokens):
        import oracle
        import stories_hip as sh
        cfg = sh.qwen3_06b_config()
        cfg.max_seq = QWEN_PROMPT + QWEN_NEW
        w = sh.synth_weights(cfg, seed=3, std=0.02).rounded(sh.SH_DTYPE_BF16)
        prompt = sh.synth_tokens(QWEN_PROMPT, 3, cfg.vocab)
        dec = oracle.Decoder(oracle.config_from(cfg), w, threads=1)
        t0 = time.perf_counter()
        toks, _, _ = dec.greedy_decode(prompt, QWEN_CPU_NEW)
        dt = time.perf_counter() - t0
        forwards = len(toks) - 1
        return {"value": round(forwards / dt, 3), "unit": "token forwards/s", "cores": 1, "kind": "port",
                "sample": f"{len(prompt)}-id prompt + {QWEN_CPU_NEW} new tokens of the same decode "
                          f"({forwards} token forwards, the oracle decoder, 1 thread, {dt:.2f} s)",
                "tokens_match_gpu": toks.tolist() == gpu_tokens[:len(toks)]}

    return decode_line(r, args.steps, "batch-1 decode tokens/sec (Qwen3-0.6B-shaped)",
                       "Qwen3-0.6B-shaped bf16 batch-1 greedy decode, 32-id prompt + 256 new tokens", "bf16",
                       "synthetic: N(0,0.02) weights seed 3 (bf16), 32-id prompt seed 3",
                       {"layers": 28, "dim": 1024, "heads": 16, "kv_heads": 8, "head_dim": 128,
                        "hidden": 3072, "vocab": 151936, "batch": 1, "prompt_tokens": QWEN_PROMPT,
                        "new_tokens": QWEN_NEW, "kv_cache": "bf16", "parallelism": "none (1 GPU)"},
                       None if args.no_cpu_baseline else cpu, TRAFFIC_QWEN)


PREFILL_S = 256
MFMA_PEAK_TFLOPS = 2500.0


def workload_prefill(args):
    r = run_cli(["-shape", "stories110m", "-dtype", "fp16", "-synthetic-seed", "0",
                 "-synthetic-std", "0.02", "-eval-logits", "-prompt-len", PREFILL_S, "-prompt-seed", "2",
                 "-bench-steps", args.steps, "-bench-warmup", args.warmup])
    steps = r["steps"]
    gpu_ms = sum(r["gpu_ms"]) / steps
    tflops = r["flops"] / (gpu_ms / 1e3) / 1e12
    line = {
        "metric": "EvalLogits full-sequence forward tokens/sec (Stories110M, S=256)",
        "value": round(PREFILL_S * steps / r["wall_s"], 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": steps, "warmup": r["warmup"], "ms_per_step": round(r["wall_s"] * 1e3 / steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic: N(0,0.02) weights seed 0 (fp16), 256 ids seed 2",
        "config": {"workload": "Stories110M EvalLogits forward, S=256, residual scale 1/sqrt(24)",
                   "layers": 12, "dim": 768, "vocab": 32000, "seq": PREFILL_S, "parallelism": "none (1 GPU)"},
        "roofline": {
            "kernel": "the forward's kernels together (MFMA GEMMs, MFMA attention, row kernels)",
            "bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tflops / MFMA_PEAK_TFLOPS, 4), "traffic": None,
            "flops_per_forward": r["flops"], "forward_ms": round(gpu_ms, 4),
        },
    }
    if not args.no_cpu_baseline:
        import oracle
        import stories_hip as sh
        cfg = sh.stories110m_config()
        cfg.residual_scale = 1.0 / (24.0 ** 0.5)
        w = sh.synth_weights(cfg, seed=0, std=0.02).rounded(sh.SH_DTYPE_F16)
        toks = sh.synth_tokens(PREFILL_S, 2, cfg.vocab)
        th = host_threads()
        oc = oracle.config_from(cfg)
        # as the reference runs it: linearCF and causalAttentionCF serial (forward_common.go:
        # 5-46), the vocabulary product over the host threads (cpu.go:276-300)
        t0 = time.perf_counter()
        logits = oracle.eval_logits_cf(oc, w, toks, threads=th, reference_threading=True)
        dt = time.perf_counter() - t0
        # every product over the host threads (not the reference's threading), for comparison
        t0 = time.perf_counter()
        oracle.eval_logits_cf(oc, w, toks, threads=th)
        dt_all = time.perf_counter() - t0
        line["cpu_baseline"] = {
            "value": round(PREFILL_S / dt, 2), "unit": "tokens/s", "cores": th, "kind": "port",
            "sample": (f"the full forward once (C restatement of engine.go:804-842) with the reference's "
                       f"threading: linearCF and attention on 1 thread, the vocabulary product on {th} "
                       f"({dt:.2f} s)"),
            "value_all_products_threaded": round(PREFILL_S / dt_all, 2),
            "sample_all_products_threaded": f"every product on {th} threads ({dt_all:.2f} s)",
            "logits_sum_cpu": float(logits.sum(dtype="float64")), "logits_sum_gpu": r["logits_sum"],
        }
    return line


BATCH_B, BATCH_PROMPT, BATCH_NEW, BATCH_CPU_NEW = 32, 1024, 128, 2


def workload_batch(args):
    r = run_cli(["-shape", "qwen3-0.6b", "-dtype", "bf16", "-synthetic-seed", "3",
                 "-synthetic-std", "0.02", "-seq", BATCH_PROMPT + BATCH_NEW, "-batch", BATCH_B,
                 "-prompt-len", BATCH_PROMPT, "-prompt-seed", "4", "-max-new", BATCH_NEW,
                 "-bench-steps", args.steps, "-bench-warmup", args.warmup,
                 "-copy-calibrate", COPY_BYTES, "-read-calibrate", COPY_BYTES])
    steps = r["steps"]
    dec_s = sum(r["decode_ms"]) / 1e3
    pre_s = sum(r["prefill_ms"]) / 1e3
    tokens = sum(r["tokens_out"])
    step_ms = sum(r["decode_ms"]) / max(sum(r["decode_steps"]), 1)
    achieved = r["bytes_per_step_mean"] / (step_ms / 1e3) / 1e9
    line = {
        "metric": "batched decode tokens/sec, aggregate (Qwen3-0.6B-shaped, 32 sequences)",
        "value": round(tokens / dec_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "ms_per_step": round(r["wall_s"] * 1e3 / steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: N(0,0.02) weights seed 3 (bf16), 32 prompts of 1024 ids seed 4",
        "config": {"workload": "Qwen3-0.6B-shaped batched greedy decode, 32 x (1024-id prompt + 128 steps)",
                   "layers": 28, "dim": 1024, "vocab": 151936, "batch": BATCH_B, "prompt_tokens": BATCH_PROMPT,
                   "new_tokens": BATCH_NEW, "kv_cache": "bf16", "parallelism": "none (1 GPU)"},
        "job_tokens_per_s_with_prefill": round(tokens / (dec_s + pre_s), 1),
        "prefill_ms": round(pre_s * 1e3 / steps, 3),
        "roofline": {
            "kernel": "one decode step's kernels together (captured graph)", "bound": "hbm",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "bytes_per_step": r["bytes_per_step_mean"], "step_ms": round(step_ms, 4),
            "copy_gbs": round(r["copy_gbs"], 1), "read_gbs": round(r["read_gbs"], 1),
        },
    }
    if not args.no_cpu_baseline:
        import oracle
        import stories_hip as sh
        cfg = sh.qwen3_06b_config()
        cfg.max_seq = BATCH_PROMPT + BATCH_NEW
        w = sh.synth_weights(cfg, seed=3, std=0.02).rounded(sh.SH_DTYPE_BF16)
        prompt = sh.synth_tokens(BATCH_B * BATCH_PROMPT, 4, cfg.vocab)[:16]
        dec = oracle.Decoder(oracle.config_from(cfg), w, threads=1)
        t0 = time.perf_counter()
        toks, _, _ = dec.greedy_decode(prompt, BATCH_CPU_NEW)
        dt = time.perf_counter() - t0
        forwards = len(toks) - 1
        line["cpu_baseline"] = {
            "value": round(forwards / dt, 3), "unit": "token forwards/s", "cores": 1, "kind": "port",
            "sample": f"one sequence: the first 16 ids of prompt 0 + {BATCH_CPU_NEW} new tokens "
                      f"({forwards} token forwards of the oracle decoder, 1 thread, {dt:.2f} s); a CPU "
                      f"decodes the 32 sequences one forward at a time",
        }
    return line


TRAIN_S = 256
MFMA_F32_PEAK_TFLOPS = 157.3


def workload_train(args):
    r = run_cli(["-shape", "stories110m", "-synthetic-seed", "0", "-synthetic-std", "0.02", "-train",
                 "-seq", TRAIN_S, "-prompt-seed", "5", "-bench-steps", args.steps, "-bench-warmup", args.warmup])
    steps = r["steps"]
    step_ms = sum(r["step_ms"]) / steps
    tflops = r["flops"] / (step_ms / 1e3) / 1e12
    line = {
        "metric": "training tokens/sec (Stories110M Engine.Step, S=256)",
        "value": round(TRAIN_S * steps / r["wall_s"], 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps,
        "warmup": r["warmup"], "ms_per_step": round(r["wall_s"] * 1e3 / steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic: N(0,0.02) fp32 weights seed 0, 65536-id token stream seed 5, drand48 windows seed 42",
        "config": {"workload": "Stories110M training step (forward, cross-entropy, backward, Adam), S=256",
                   "layers": 12, "dim": 768, "vocab": 32000, "seq": TRAIN_S, "lr": 3e-4, "loss_scale": 256,
                   "parallelism": "none (1 GPU)"},
        "loss_first_last": [r["loss"][0], r["loss"][-1]],
        "roofline": {
            "kernel": "the step's kernels together (fp32 MFMA GEMMs, attention, row kernels, Adam)",
            "bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_F32_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tflops / MFMA_F32_PEAK_TFLOPS, 4), "traffic": None,
            "flops_per_step": r["flops"], "step_ms": round(step_ms, 4),
        },
    }
    if not args.no_cpu_baseline:
        import oracle
        import stories_hip as sh
        cfg = sh.stories110m_config()
        cfg.residual_scale = 1.0 / (24.0 ** 0.5)
        w = sh.synth_weights(cfg, seed=0, std=0.02)
        p = oracle.TrainParams.from_weights(w)
        m, v, g = (oracle.TrainParams.zeros_like(p) for _ in range(3))
        stream = sh.synth_tokens(1 << 16, 5, cfg.vocab).astype("uint16")
        L = oracle.load()
        st = oracle.C.c_uint64(L.or_drand48_seed(42))
        pos = L.or_train_window(oracle.C.byref(st), stream.size, TRAIN_S)
        th = host_threads()
        t0 = time.perf_counter()
        loss = oracle.train_step(oracle.config_from(cfg), p, m, v, g, oracle.hparams(), 1,
                                 stream[pos:pos + TRAIN_S], stream[pos + 1:pos + 1 + TRAIN_S], threads=th)
        dt = time.perf_counter() - t0
        line["cpu_baseline"] = {
            "value": round(TRAIN_S / dt, 2), "unit": "tokens/s", "cores": th, "kind": "port",
            "sample": f"the first step of the same run (C restatement of train_full.go's CPU path, {th} threads, "
                      f"{dt:.2f} s)",
            "loss_cpu": loss,
        }
    return line


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "prefill", "w8a8", "qwen-decode", "batch", "train"])
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "this build has no multi-GPU path", file=sys.stderr)
        return 2
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    if args.workload != "decode":
        fn = {"prefill": workload_prefill, "w8a8": workload_w8a8, "qwen-decode": workload_qwen_decode,
              "batch": workload_batch, "train": workload_train}[args.workload]
        print(json.dumps(with_host(fn(args))))
        return 0

    r = gpu_leg(args.steps, args.warmup)
    steps = r["steps"]
    gen_tokens = sum(r["generated"])
    forwards = sum(r["forwards"])
    # each decode's device time = the prompt's cache-filling forward (full-sequence kernels)
    # + the token loop (one k_decode_persistent launch); the roofline is the launch's
    prefill_ms = sum(r.get("prefill_ms", [0.0] * steps))
    gpu_ms = sum(r["gpu_ms"]) - prefill_ms
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
            "prompt_forward_ms": round(prefill_ms / steps, 4),
            "copy_gbs": round(r["copy_gbs"], 1),
            "read_gbs": round(r["read_gbs"], 1),
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(r["tokens"])
    print(json.dumps(with_host(line)))
    return 0


if __name__ == "__main__":
    sys.exit(main())
