"""GPU parity of the full-sequence forward (EvalLogits, engine.go:804-842) against the CPU
oracle's channel-first restatement, through the C ABI.

Bar: logits [V, S] within max-abs 2e-2 of the oracle fed the same dtype-rounded weights.
The GPU feeds its MFMA GEMMs hi/lo planes of the fp32 activations, so the measured errors
sit near 1e-5; the bar is the float one.
"""
import math
import os

import numpy as np
import pytest

import oracle
import stories_hip as sh
from helpers import random_gains, tiny_config, tiny_gqa_config

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2
THREADS = max(1, min(16, os.cpu_count() or 1))


def build(cfg, dtype, seed, std=0.02, gains_seed=None):
    w = sh.synth_weights(cfg, seed=seed, std=std)
    if gains_seed is not None:
        w = random_gains(w, gains_seed)
    m = sh.Model(cfg, dtype)
    m.upload(w)
    return m, oracle.config_from(cfg), w.rounded(dtype)


def compare(m, ocfg, ow, tokens, tol=LOGIT_TOL):
    got = m.eval_logits(tokens)
    want = oracle.eval_logits_cf(ocfg, ow, tokens, threads=THREADS)
    assert got.shape == want.shape == (ocfg.vocab, len(tokens))
    err = float(np.max(np.abs(got - want)))
    scale = float(np.max(np.abs(want)))
    print(f"S={len(tokens)}: max-abs {err:.3e} (max |logit| {scale:.3f}), "
          f"{m.stats()['gpu_ms']:.3f} ms")
    assert err <= tol, err
    return got, want, err


@pytest.mark.parametrize("seq", [1, 17, 64])
def test_prefill_tiny_fp16(gpu, seq):
    cfg = tiny_config()
    m, ocfg, ow = build(cfg, sh.SH_DTYPE_F16, seed=201, std=0.08, gains_seed=202)
    toks = sh.synth_tokens(seq, 203 + seq, cfg.vocab)
    compare(m, ocfg, ow, toks)
    m.close()


def test_prefill_tiny_residual_scale_and_bad_ids(gpu):
    """alpha = 1/sqrt(2L) (engine.go residual path) and out-of-range ids (zero columns)."""
    cfg = tiny_config(n_layers=3, residual_scale=1.0 / math.sqrt(6.0))
    m, ocfg, ow = build(cfg, sh.SH_DTYPE_F16, seed=211, std=0.08)
    toks = sh.synth_tokens(33, 212, cfg.vocab).astype(np.int64)
    toks[[0, 5, 31]] = [cfg.vocab, cfg.vocab + 7, 65535]
    compare(m, ocfg, ow, toks)
    m.close()


def test_prefill_tiny_gqa_qknorm_bf16(gpu):
    cfg = tiny_gqa_config()
    m, ocfg, ow = build(cfg, sh.SH_DTYPE_BF16, seed=221, std=0.08, gains_seed=222)
    compare(m, ocfg, ow, sh.synth_tokens(48, 223, cfg.vocab))
    m.close()


def test_prefill_repeat_and_shrink(gpu):
    """Scratch is reused across calls: a longer then a shorter sequence, then the first again."""
    cfg = tiny_config()
    m, ocfg, ow = build(cfg, sh.SH_DTYPE_F16, seed=231, std=0.08)
    a = sh.synth_tokens(40, 232, cfg.vocab)
    first = m.eval_logits(a)
    compare(m, ocfg, ow, a[:9])
    np.testing.assert_array_equal(m.eval_logits(a), first)
    with pytest.raises(sh.ShError):
        m.eval_logits(np.zeros(cfg.max_seq + 1, np.uint16))
    m.close()


def test_prefill_graph_replays_match_oracle(gpu):
    """The forward runs as one captured graph, replayed while the length stays the same:
    three calls of one length with different ids, eager decode steps between them, each
    against the oracle."""
    cfg = tiny_config()
    m, ocfg, ow = build(cfg, sh.SH_DTYPE_F16, seed=251, std=0.08, gains_seed=252)
    for r in range(3):
        toks = sh.synth_tokens(33, 253 + r, cfg.vocab)
        compare(m, ocfg, ow, toks)
        m.reset_cache()
        m.eval_next_logits(int(toks[0]), 0)
    m.close()


def test_prefill_columns_match_kv_cache_decode(gpu):
    """Column t of the causal forward equals the KV-cache decode at position t (two GPU
    paths with different kernels), and both match the oracle."""
    cfg = tiny_config()
    m, ocfg, ow = build(cfg, sh.SH_DTYPE_F16, seed=241, std=0.08, gains_seed=242)
    toks = sh.synth_tokens(24, 243, cfg.vocab)
    pf = m.eval_logits(toks)
    m.reset_cache()
    for t, tok in enumerate(toks):
        lg, _ = m.eval_next_logits(int(tok), t)
        assert float(np.max(np.abs(lg - pf[:, t]))) <= LOGIT_TOL
    m.close()


def test_prefill_stories110m_s256(gpu):
    """Stories110M fp16, alpha = 1/sqrt(24) (the storiesane engine's residual scale), the
    prefill configuration's input: 256 token ids uniform in [0, 32000) from seed 2; logits
    [32000, 256] within 2e-2 of the oracle."""
    cfg = sh.stories110m_config()
    cfg.residual_scale = 1.0 / math.sqrt(2.0 * cfg.n_layers)
    m, ocfg, ow = build(cfg, sh.SH_DTYPE_F16, seed=0)
    toks = sh.synth_tokens(256, 2, cfg.vocab)
    got, want, _ = compare(m, ocfg, ow, toks)
    # greedy choice per position agrees wherever the oracle's top-2 margin is clear
    top2 = np.sort(want, axis=0)[-2:]
    clear = (top2[1] - top2[0]) > 2 * LOGIT_TOL
    assert np.array_equal(np.argmax(got, axis=0)[clear], np.argmax(want, axis=0)[clear])
    m.close()


@pytest.mark.parametrize("gqa", [False, True])
def test_prefill_wide_attention_tails(gpu, gqa):
    """2050 positions of a 12-head model (4 kv heads with GQA): the 64-query attention form
    (ceil(S/64) x H >= 256 workgroups) with a partial last chunk of query blocks (33 = 2 x 16
    + 1) and a grid of 396 workgroups (not a multiple of the 8 XCDs), and the 128 x 128 burst
    GEMMs with a partial last group of row tiles (17 = 2 x 8 + 1), W2 split into two K
    ranges: every tile of both XCD-grouped orders is computed once and lands where the oracle
    puts it."""
    shape = dict(dim=384, hidden=512, n_heads=12, n_kv_heads=4 if gqa else 12, max_seq=2112)
    cfg = (tiny_gqa_config if gqa else tiny_config)(**shape)
    dtype = sh.SH_DTYPE_BF16 if gqa else sh.SH_DTYPE_F16
    # (fp16 takes the activations as one fp16 plane: weights of std 0.02 keep its logits, and
    # with them its rounding, at the scale of the models it serves)
    m, ocfg, ow = build(cfg, dtype, seed=221 + gqa, std=0.08 if gqa else 0.02, gains_seed=223)
    compare(m, ocfg, ow, sh.synth_tokens(2050, 224 + gqa, cfg.vocab))
    m.close()


def test_prefill_qwen3_shaped_bf16(gpu):
    """Qwen3-0.6B-shaped bf16 (GQA 16/8, hd 128, QK-norm, theta 1e6), 64 tokens."""
    cfg = sh.qwen3_06b_config()
    m, ocfg, ow = build(cfg, sh.SH_DTYPE_BF16, seed=3)
    compare(m, ocfg, ow, sh.synth_tokens(64, 7, cfg.vocab))
    m.close()


def test_prefill_long_then_short_reuses_scratch(gpu):
    """A long input (128 x 128 tiles, K not split) then a short one on the same model (64 x 64
    tiles, K split into ranges): the second call needs more K-range scratch than the first
    allocated, and must equal the same call on a fresh model."""
    cfg = sh.qwen3_06b_config()
    w = sh.synth_weights(cfg, seed=3, std=0.02)
    m = sh.Model(cfg, sh.SH_DTYPE_BF16)
    m.upload(w)
    m.eval_logits(sh.synth_tokens(1100, 8, cfg.vocab))
    short = sh.synth_tokens(48, 9, cfg.vocab)
    got = m.eval_logits(short)
    m.close()
    fresh = sh.Model(cfg, sh.SH_DTYPE_BF16)
    fresh.upload(w)
    np.testing.assert_array_equal(got, fresh.eval_logits(short))
    fresh.close()
