"""GPU parity of the W8A8 decode (int8 weights per output row, int8 activations per tensor,
int32 accumulation; the bridge quantizer of ane_bridge.m:374-399 applied to every projection
and the classifier) against the oracle's W8A8 decoder, through the C ABI.

Bars: logits within max-abs 2e-2; greedy token streams identical. The int32 dot products
are exact on both sides, so differences come only from fp32 rounding upstream of an
activation quantization (a different sum order can move x/s across a .5 boundary)."""
import os

import numpy as np
import pytest

import oracle
import stories_hip as sh
from helpers import random_gains, tiny_config, tiny_gqa_config

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2
THREADS = max(1, min(16, os.cpu_count() or 1))


def build(cfg, seed, std=0.02, gains_seed=None):
    w = sh.synth_weights(cfg, seed=seed, std=std)
    if gains_seed is not None:
        w = random_gains(w, gains_seed)
    m = sh.Model(cfg, sh.SH_DTYPE_W8A8)
    m.upload(w)
    print(m.describe())
    ref = oracle.Decoder(oracle.config_from(cfg, w8a8=True), w.rounded(sh.SH_DTYPE_W8A8),
                         threads=THREADS)
    return m, ref


def check_steps(m, ref, tokens):
    worst = 0.0
    for pos, tok in enumerate(tokens):
        got, am = m.eval_next_logits(int(tok), pos)
        want = ref.forward_one(int(tok), pos)
        err = float(np.max(np.abs(got - want)))
        worst = max(worst, err)
        assert err <= LOGIT_TOL, f"pos {pos}: max-abs {err}"
        assert am == int(np.argmax(got))
    print(f"W8A8 max-abs logits error over {len(tokens)} positions: {worst:.3e}")
    return worst


@pytest.mark.parametrize("kv", [sh.SH_KV_F32, sh.SH_KV_F16])
def test_w8a8_decode_step_tiny(gpu, kv):
    cfg = tiny_config(kv_dtype=kv)
    m, ref = build(cfg, seed=401, std=0.08, gains_seed=402)
    check_steps(m, ref, sh.synth_tokens(40, 403, cfg.vocab))
    p = sh.synth_tokens(6, 404, cfg.vocab)
    got, _, _ = m.greedy_decode(p, 30)
    want, _, _ = ref.greedy_decode(p, 30)
    assert got.tolist() == want.tolist()
    assert m.stats()["persistent"]
    m.close()


def test_w8a8_tiny_gqa_qknorm(gpu):
    cfg = tiny_gqa_config()
    m, ref = build(cfg, seed=411, std=0.08, gains_seed=412)
    check_steps(m, ref, sh.synth_tokens(32, 413, cfg.vocab))
    m.close()


def test_w8a8_shape_without_persistent_kernel_is_rejected(gpu):
    cfg = tiny_config(dim=256, hidden=512, n_heads=8, n_kv_heads=4, head_dim=32)
    with pytest.raises(sh.ShError, match="W8A8"):
        sh.Model(cfg, sh.SH_DTYPE_W8A8)


def test_stories110m_w8a8_greedy_128(gpu):
    """Stories110M W8A8: per-row int8 of the seed-0 N(0, 0.02) weights, 16-id prompt from
    seed 1, 128 new tokens; identical token stream, logits within 2e-2."""
    cfg = sh.stories110m_config()
    m, ref = build(cfg, seed=0)
    prompt = sh.synth_tokens(16, 1, cfg.vocab)
    got, plen, eos = m.greedy_decode(prompt, 128)
    want, weos, margins = ref.greedy_decode(prompt, 128)
    print(f"generated {len(got) - plen} tokens; smallest top-2 margin {np.nanmin(margins):.3e}")
    assert got.tolist() == want.tolist() and eos == weos
    st = m.stats()
    print(f"persistent={st['persistent']} grid={st['grid']} {st['gpu_ms']:.3f} ms for "
          f"{st['forwards']} forwards, {st['bytes_per_forward_mean'] / 1e6:.2f} MB/forward")
    assert st["persistent"]
    m.reset_cache()
    ref.reset()
    check_steps(m, ref, got[:24])
    m.close()
