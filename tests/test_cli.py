"""The stories-generate host program (cmd/stories-generate-go/main.go counterpart): llama2.c
model and tokenizer file readers and flag handling on the CPU (-inspect / -detokenize touch
no GPU); greedy and sampled decodes through the C ABI on the GPU."""
import json
import os
import subprocess

import numpy as np
import pytest

import oracle
import stories_hip as sh
from helpers import (BLZT_LAYER_ORDER, LLAMA2_ORDER, deepnet_alpha, splitmix64_uniforms, tiny_config, write_blzt,
                     write_llama2_bin, write_tokenizer_bin)

CLI = os.path.join(os.path.dirname(sh.LIB_PATH), "stories-generate")
LOGIT_TOL = 2e-2  # max-abs logits bar


def run(*args, check=True):
    if not os.path.exists(CLI):
        pytest.fail(f"{CLI} is not built (make -C ane-training-experiments_amd)")
    p = subprocess.run([CLI, *map(str, args)], capture_output=True, text=True, timeout=300)
    if check and p.returncode != 0:
        raise AssertionError(f"exit {p.returncode}: {p.stderr}")
    return p


def distinct_weights(cfg, seed):
    """Weights whose tensors all have different sums, so a swapped read order shows."""
    w = sh.synth_weights(cfg, seed=seed, std=0.05)
    for l, lw in enumerate(w.layers):
        for j, k in enumerate(LLAMA2_ORDER):
            lw[k] = (lw[k] + np.float32(0.001 * (1 + j + 10 * l))).astype(np.float32)
    w.rms_final = (w.rms_final * np.float32(1.5)).astype(np.float32)
    return w


def gqa_file_config():
    return tiny_config(n_heads=4, n_kv_heads=2, max_seq=64)


def test_inspect_reads_llama2_layout(tmp_path):
    cfg = gqa_file_config()
    w = distinct_weights(cfg, 301)
    path = tmp_path / "m.bin"
    write_llama2_bin(path, cfg, w)
    got = json.loads(run("-model", path, "-inspect").stdout)
    assert got["header"] == {"dim": 128, "hidden": 256, "n_layers": 2, "n_heads": 4,
                             "n_kv_heads": 2, "vocab": 512, "seq_len": 64}
    assert got["shared_classifier"] is True
    want = {"embed": w.embed, "rms_final": w.rms_final}
    for k in LLAMA2_ORDER:
        want[k] = np.concatenate([lw[k].ravel() for lw in w.layers])
    for k, v in want.items():
        assert got["sums"][k] == pytest.approx(float(np.sum(v, dtype=np.float64)), rel=1e-12, abs=1e-12), k


def test_inspect_negative_vocab_and_errors(tmp_path):
    cfg = gqa_file_config()
    w = distinct_weights(cfg, 302)
    path = tmp_path / "neg.bin"
    write_llama2_bin(path, cfg, w, negative_vocab=True)
    got = json.loads(run("-model", path, "-inspect").stdout)
    assert got["header"]["vocab"] == -512 and got["shared_classifier"] is False
    # truncated inside layer 1's w3: the error names the tensor (weights.go:116-118)
    data = path.read_bytes()
    cut = tmp_path / "cut.bin"
    cut.write_bytes(data[:len(data) - 4 * cfg.dim - 100])
    p = run("-model", cut, "-inspect", check=False)
    assert p.returncode == 1 and "read w3[1]: unexpected EOF" in p.stderr
    cut.write_bytes(data[:20])
    p = run("-model", cut, "-inspect", check=False)
    assert p.returncode == 1 and "read config: unexpected EOF" in p.stderr
    bad = tmp_path / "bad.bin"
    bad.write_bytes(np.array([128, 256, 2, 5, 5, 512, 64], "<i4").tobytes())
    p = run("-model", bad, "-inspect", check=False)
    assert p.returncode == 1 and "config mismatch" in p.stderr
    p = run("-model", tmp_path / "missing.bin", "-inspect", check=False)
    assert p.returncode == 1 and "open" in p.stderr


@pytest.mark.parametrize("version", [2, 3])
def test_inspect_reads_blzt_checkpoint(tmp_path, version):
    cfg = tiny_config(max_seq=64)
    w = distinct_weights(cfg, 305)
    for lw in w.layers:
        lw["rms_att"] = (lw["rms_att"] * np.float32(1.25)).astype(np.float32)
    path = tmp_path / "c.bin"
    write_blzt(path, cfg, w, version=version)
    got = json.loads(run("-ckpt", path, "-inspect").stdout)
    ck = got["checkpoint"]
    assert (ck["version"], ck["step"], ck["total_steps"], ck["n_layers"], ck["vocab"], ck["dim"],
            ck["hidden"], ck["heads"], ck["seq"]) == (version, 7, 100, 2, 512, 128, 256, 4, 64)
    assert ck["lr"] == pytest.approx(3e-4) and ck["loss"] == 2.5 and ck["cum_wall"] == 3.75
    assert (ck["cum_steps"], ck["cum_batches"], ck["adam_t"]) == (6, 12, 7)
    want = {"embed": w.embed, "rms_final": w.rms_final}
    for k in BLZT_LAYER_ORDER:
        want[k] = np.concatenate([lw[k].ravel() for lw in w.layers])
    for k, v in want.items():
        assert got["sums"][k] == pytest.approx(float(np.sum(v, dtype=np.float64)), rel=1e-12, abs=1e-12), k


def test_blzt_errors(tmp_path):
    cfg = tiny_config(max_seq=64)
    w = distinct_weights(cfg, 306)
    path = tmp_path / "c.bin"
    write_blzt(path, cfg, w, version=3)
    data = path.read_bytes()
    bad = tmp_path / "bad.bin"
    bad.write_bytes(data[:4] + np.array([4], "<i4").tobytes() + data[8:])
    p = run("-ckpt", bad, "-inspect", check=False)
    assert p.returncode == 1 and "bad checkpoint header magic=424c5a54 version=4" in p.stderr
    bad.write_bytes(np.array([0x12345678], "<i4").tobytes() + data[4:])
    p = run("-ckpt", bad, "-inspect", check=False)
    assert p.returncode == 1 and "bad checkpoint header magic=12345678" in p.stderr
    hdr = np.frombuffer(data[:40], "<i4").copy()
    hdr[8] = 5                                     # heads not dividing dim
    bad.write_bytes(hdr.tobytes() + data[40:])
    p = run("-ckpt", bad, "-inspect", check=False)
    assert p.returncode == 1 and "checkpoint config mismatch" in p.stderr
    for cut, what in ((len(data) - 8, "embed optimizer state"), (len(data) - 2 * 512 * 128 * 4 - 100, "embed"),
                      (200, "wq[0]")):
        bad.write_bytes(data[:cut])
        p = run("-ckpt", bad, "-inspect", check=False)
        assert p.returncode == 1 and what in p.stderr and "unexpected EOF" in p.stderr, (what, p.stderr)


def test_detokenize(tmp_path):
    pieces = ["<unk>", "<s>", "</s>"] + [f"p{i}" for i in range(3, 32000)]
    pieces[65] = "<0x41>"      # byte token -> "A"
    pieces[66] = "<0x0a>"      # lowercase hex -> "\n"
    pieces[67] = "<0xZZ>"      # not hex: kept literally
    pieces[68] = "<0x4>"       # wrong length: kept literally
    pieces[69] = " world"
    path = tmp_path / "tok.bin"
    write_tokenizer_bin(path, pieces)
    p = run("-tokenizer", path, "-detokenize", "65,69,66,67,68,-1,32000,5")
    assert p.stdout == "text=A world\n<0xZZ><0x4>p5\n"
    bad = tmp_path / "bad.bin"
    write_tokenizer_bin(bad, pieces, max_len=0)
    p = run("-tokenizer", bad, "-detokenize", "5", check=False)
    assert p.returncode == 1 and "bad tokenizer header: max token len=0" in p.stderr
    short = tmp_path / "short.bin"
    write_tokenizer_bin(short, pieces[:100])
    p = run("-tokenizer", short, "-detokenize", "5", check=False)
    assert p.returncode == 1 and "unexpected EOF at token 100" in p.stderr


def test_flag_errors(tmp_path):
    p = run("-no-such-flag", "1", check=False)
    assert p.returncode == 1 and "flag provided but not defined: -no-such-flag" in p.stderr
    p = run("-prompt-ids", "1,x", "-inspect", check=False)
    assert p.returncode == 1
    cfg = gqa_file_config()
    path = tmp_path / "m.bin"
    write_llama2_bin(path, cfg, sh.synth_weights(cfg, seed=1, std=0.05))
    p = run("-model", path, "-batch", "2", check=False)
    assert p.returncode == 1 and "-batch needs -bench-steps and -prompt-len" in p.stderr
    p = run("-model", path, "-eval-logits", "-bench-steps", "2", check=False)
    assert p.returncode == 1 and "-eval-logits needs -bench-steps and -prompt-len" in p.stderr


# ---- GPU ---------------------------------------------------------------------------------

@pytest.mark.gpu
def test_cli_greedy_decode_of_llama2_file_matches_oracle(tmp_path):
    """-model file, -temperature 0: the token stream equals the oracle's greedy decode of the
    same file weights (fp16-rounded), config from the file header (theta 1e4, eps 1e-5)."""
    cfg = gqa_file_config()
    w = sh.synth_weights(cfg, seed=311, std=0.08)
    path = tmp_path / "m.bin"
    write_llama2_bin(path, cfg, w)
    p = run("-model", path, "-prompt-ids", "5, 9,11", "-max-new", "40", "-temperature", "0",
            "-seq", "64", "-seed", "1")
    lines = p.stdout.splitlines()
    assert lines[0].startswith("source=pretrained prompt_tokens=3 ")
    got = [int(t) for t in lines[1].split("=", 1)[1].split(",")]
    assert lines[2] == "text=(tokenizer not provided)"
    ref = oracle.Decoder(oracle.config_from(cfg), w.rounded(sh.SH_DTYPE_F16), threads=4)
    want, eos, _ = ref.greedy_decode([5, 9, 11], 40)
    assert got == want.tolist()
    assert f"generated_tokens={len(got) - 3} " in lines[0] and f"eos={'true' if eos else 'false'}" in lines[0]
    # the device-side rate fields follow main.go:60-67's line
    fields = dict(kv.split("=", 1) for kv in lines[0].split())
    assert float(fields["hbm_gbps"]) > 0 and 0 < float(fields["roofline_frac"]) < 1


@pytest.mark.gpu
def test_cli_sampled_decode_is_seeded(tmp_path):
    """-temperature 0.8: ids drawn on the host from device logits; the same -seed gives the
    same stream (the reference's math/rand stream itself is not reproduced)."""
    cfg = gqa_file_config()
    path = tmp_path / "m.bin"
    write_llama2_bin(path, cfg, sh.synth_weights(cfg, seed=321, std=0.08))
    a = run("-model", path, "-prompt-ids", "1", "-max-new", "30", "-temperature", "0.8",
            "-seq", "64", "-seed", "7").stdout.splitlines()[1]
    b = run("-model", path, "-prompt-ids", "1", "-max-new", "30", "-temperature", "0.8",
            "-seq", "64", "-seed", "7").stdout.splitlines()[1]
    assert a == b
    ids = [int(t) for t in a.split("=", 1)[1].split(",")]
    assert all(0 <= t < cfg.vocab for t in ids) and len(ids) >= 2


def cli_ids(stdout):
    return [int(t) for t in stdout.splitlines()[1].split("=", 1)[1].split(",")]


def check_sampled_stream(ids, plen, want_logits, temp, seed, delta, what):
    """The CLI's sampled ids against sampleFromLogits (infer.go:347-371, the oracle's
    restatement) fed the oracle's logits at each step of the CLI's own stream and the same
    splitmix64 draws. The device logits are within delta of the oracle's, which moves every
    normalised CDF boundary by at most 4 (e^(2 delta / T) - 1); where the draw lies farther
    than that from its interval's ends the ids must be equal (pinned), elsewhere they may
    differ. Returns the number of pinned steps."""
    draws = splitmix64_uniforms(seed, len(want_logits))
    bound = 4.0 * (np.exp(2.0 * delta / temp) - 1.0) + 1e-12
    pinned = 0
    for k, lg in enumerate(want_logits):
        idx, slack = oracle.sample_from_logits(lg, temp, float(draws[k]))
        if slack > bound:
            pinned += 1
            assert ids[plen + k] == idx, f"{what}: step {k}: CLI {ids[plen + k]}, oracle sampler {idx}"
    print(f"{what}: {pinned} of {len(want_logits)} steps pinned (delta {delta:.2e}, bound {bound:.2e})")
    return pinned


@pytest.mark.gpu
def test_cli_sampled_decode_matches_oracle_sampler(tmp_path):
    """-temperature 0.8 on the KV-cache decoder: every pinned step's id equals the oracle
    sampler's (check_sampled_stream), the oracle teacher-forced on the CLI's stream and the
    draws the CLI's documented splitmix64 stream seeded by -seed (Go's math/rand stream itself
    is not reproduced). delta is measured through the library on the same stream."""
    cfg = gqa_file_config()
    w = sh.synth_weights(cfg, seed=331, std=0.08)
    path = tmp_path / "m.bin"
    write_llama2_bin(path, cfg, w)
    temp, seed, plen = 0.8, 7, 3
    ids = cli_ids(run("-model", path, "-prompt-ids", "5,9,11", "-max-new", "40", "-temperature", temp,
                      "-seq", "64", "-seed", seed).stdout)
    ref = oracle.Decoder(oracle.config_from(cfg), w.rounded(sh.SH_DTYPE_F16), threads=4)
    m = sh.Model(cfg, sh.SH_DTYPE_F16)
    m.upload(w)
    want, delta = [], 0.0
    for pos in range(len(ids) - 1):
        lo = ref.forward_one(ids[pos], pos)
        lg, _ = m.eval_next_logits(ids[pos], pos)
        delta = max(delta, float(np.max(np.abs(lg - lo))))
        if pos >= plen - 1:
            want.append(lo)
    m.close()
    assert len(want) == len(ids) - plen
    assert check_sampled_stream(ids, plen, want, temp, seed, delta, "KV decoder") >= 0.9 * len(want)


@pytest.mark.gpu
def test_cli_ane_decode_matches_window_oracle(tmp_path):
    """-ane (main.go:71-85: storiesane.Open + (*Engine).Decode, decode.go:18-94): the window of
    the last -seq ids, BOS-padded, evaluated whole every step with the engine's residual scale
    1/sqrt(2 L). -temperature 0: the ids equal the oracle's window decode (engine.go:804-842
    per step, first maximum of the last column). -temperature 0.8: every pinned step's id
    equals the oracle sampler's on the oracle's window logits of the CLI's own stream, with the
    engine's draws seeded by -seed (42 when it is 0, engine.go:166-168)."""
    cfg = gqa_file_config()
    w = sh.synth_weights(cfg, seed=341, std=0.08)
    path = tmp_path / "m.bin"
    write_llama2_bin(path, cfg, w)
    seq = 16
    acfg = tiny_config(n_heads=4, n_kv_heads=2, max_seq=seq, residual_scale=deepnet_alpha(cfg.n_layers))
    ocfg, ow = oracle.config_from(acfg), w.rounded(sh.SH_DTYPE_F16)
    # greedy: the window slides past 16 tokens
    p = run("-ane", "-model", path, "-prompt-ids", "5,9,11", "-max-new", "24", "-temperature", "0", "-seq", seq)
    assert p.stdout.splitlines()[0].startswith("source=pretrained prompt_tokens=3 ")
    got = cli_ids(p.stdout)
    toks = [5, 9, 11]
    while len(toks) < len(got):
        window = oracle.fill_decode_window(seq, np.asarray(toks, np.int32))
        toks.append(int(np.argmax(oracle.eval_logits_cf(ocfg, ow, window, threads=4)[:, seq - 1])))
        if toks[-1] == 2:
            break
    assert got == toks and (len(got) == 3 + 24 or got[-1] == 2)
    # sampled, seed 0 -> 42
    temp, plen = 0.8, 3
    ids = cli_ids(run("-ane", "-model", path, "-prompt-ids", "5,9,11", "-max-new", "20", "-temperature", temp,
                      "-seq", seq, "-seed", 0).stdout)
    # The sampler: the oracle's sampleFromLogits on the device's own EvalLogits of every window
    # of the CLI's stream, with the same draws, gives the CLI's id at every step (EvalLogits
    # carries fp16 activations, so the oracle's logits alone pin only steps far from a CDF
    # boundary); those logits are within the bar of the oracle's.
    m = sh.Model(acfg, sh.SH_DTYPE_F16)
    m.upload(w)
    draws = splitmix64_uniforms(42, len(ids) - plen)
    delta = 0.0
    for k in range(len(ids) - plen):
        window = oracle.fill_decode_window(seq, np.asarray(ids[:plen + k], np.int32))
        lo = oracle.eval_logits_cf(ocfg, ow, window, threads=4)[:, seq - 1]
        lg = m.eval_logits(window)[:, seq - 1]
        delta = max(delta, float(np.max(np.abs(lg - lo))))
        idx, _ = oracle.sample_from_logits(lg, temp, float(draws[k]))
        assert ids[plen + k] == idx, f"-ane step {k}: CLI {ids[plen + k]}, sampler on the device logits {idx}"
    m.close()
    print(f"-ane sampled: {len(ids) - plen} steps equal; logits within {delta:.2e} of the oracle")
    assert delta <= LOGIT_TOL


@pytest.mark.gpu
def test_cli_bench_mode_stories110m():
    p = run("-shape", "stories110m", "-prompt-len", "16", "-prompt-seed", "1", "-max-new", "128",
            "-bench-steps", "2", "-bench-warmup", "1")
    r = json.loads(p.stdout)
    assert r["steps"] == 2 and len(r["gpu_ms"]) == 2 and r["persistent"] == 1
    # the 15 prompt positions before the last fill the KV cache in one full-sequence forward
    # (prefill_ms); the persistent launch runs the 128 generating forwards
    assert r["forwards"] == [128, 128] and r["generated"] == [128, 128]
    assert all(0 < pm < g for pm, g in zip(r["prefill_ms"], r["gpu_ms"]))
    cfg = sh.stories110m_config()
    w = sh.synth_weights(cfg, seed=0, std=0.02)
    ref = oracle.Decoder(oracle.config_from(cfg), w.rounded(sh.SH_DTYPE_F16), threads=16)
    want, _, _ = ref.greedy_decode(sh.synth_tokens(16, 1, cfg.vocab), 128)
    assert r["tokens"] == want.tolist()


@pytest.mark.gpu
def test_cli_batch_bench_mode(tmp_path):
    """-batch: sequences decoded together; row 0's stream equals the oracle's greedy decode of
    its prompt."""
    cfg = gqa_file_config()
    w = sh.synth_weights(cfg, seed=331, std=0.08)
    path = tmp_path / "m.bin"
    write_llama2_bin(path, cfg, w)
    p = run("-model", path, "-batch", "3", "-prompt-len", "5", "-prompt-seed", "7", "-max-new", "20",
            "-bench-steps", "2", "-bench-warmup", "1", "-seq", "64")
    r = json.loads(p.stdout)
    assert r["batch"] == 3 and r["steps"] == 2 and len(r["decode_ms"]) == 2
    assert r["decode_steps"] == [20, 20] and all(v > 0 for v in r["prefill_ms"])
    ref = oracle.Decoder(oracle.config_from(cfg), w.rounded(sh.SH_DTYPE_F16), threads=4)
    prompts = sh.synth_tokens(3 * 5, 7, cfg.vocab).reshape(3, 5)
    want, _, _ = ref.greedy_decode(prompts[0], 20)
    assert r["tokens_row0"] == want.tolist()


@pytest.mark.gpu
def test_cli_decode_from_blzt_checkpoint(tmp_path):
    """-ckpt: the same weights as a llama2.c file and as a checkpoint decode to the same ids."""
    cfg = tiny_config(max_seq=64)
    w = sh.synth_weights(cfg, seed=331, std=0.08)
    ck, mb = tmp_path / "c.bin", tmp_path / "m.bin"
    write_blzt(ck, cfg, w)
    write_llama2_bin(mb, cfg, w)
    args = ("-prompt-ids", "4,5,6", "-max-new", "24", "-temperature", "0", "-seq", "64")
    a = run("-ckpt", ck, *args).stdout.splitlines()
    b = run("-model", mb, *args).stdout.splitlines()
    assert a[0].startswith("source=checkpoint") and a[1] == b[1]


@pytest.mark.gpu
def test_cli_child_while_this_process_holds_a_persistent_model(gpu, tmp_path):
    """Two processes on one GPU: this process decodes with the persistent kernel, the child
    program then runs its own persistent decode, and this process decodes again. Both must
    run the persistent kernel and agree with the oracle (the kernel is a plain launch, so
    one process's launches do not block another's)."""
    cfg = gqa_file_config()
    w = sh.synth_weights(cfg, seed=341, std=0.08)
    m = sh.Model(cfg, sh.SH_DTYPE_F16)
    m.upload(w)
    ref = oracle.Decoder(oracle.config_from(cfg), w.rounded(sh.SH_DTYPE_F16), threads=4)
    want, _, _ = ref.greedy_decode([5, 9, 11], 30)
    got, _, _ = m.greedy_decode([5, 9, 11], 30)
    assert got.tolist() == want.tolist() and m.stats()["persistent"]
    path = tmp_path / "m.bin"
    write_llama2_bin(path, cfg, w)
    p = run("-model", path, "-prompt-ids", "5,9,11", "-max-new", "30", "-temperature", "0",
            "-seq", "64")
    assert [int(t) for t in p.stdout.splitlines()[1].split("=", 1)[1].split(",")] == want.tolist()
    got, _, _ = m.greedy_decode([5, 9, 11], 30)
    assert got.tolist() == want.tolist() and m.stats()["persistent"]
    m.close()
