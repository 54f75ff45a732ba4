"""GPU parity of the W8A8 decode (int8 weights per output row, int8 activations per tensor,
int32 accumulation; the bridge quantizer of ane_bridge.m:374-399 applied to every projection
and the classifier) against the oracle's W8A8 decoder, through the C ABI.

Bars: logits within max-abs 2e-2; greedy token streams identical. The int32 dot products
are exact on both sides, so differences come only from fp32 rounding upstream of an
activation quantization (a different sum order can move x/s across a .5 boundary). The
device keeps the reference's float order wherever a result feeds a quantizer (norms in
float64, attention sums in position order), so the Stories110M decode is asserted
bit-identical: every forward's logits and the last forward's intermediates."""
import os

import numpy as np
import pytest

import oracle
import stories_hip as sh
from helpers import oracle_stream, random_gains, tiny_config, tiny_gqa_config, top2_margins

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
    seed 1, 128 new tokens; identical token stream, and the logits of all 143 forwards
    bit-identical to the oracle's; then the last forward's intermediates (sh_decode_tap,
    the counterpart of the engine's cache taps, engine_test.go:154-239) equal the oracle's
    bit for bit."""
    cfg = sh.stories110m_config()
    m, ref = build(cfg, seed=0)
    prompt = sh.synth_tokens(16, 1, cfg.vocab)
    got, plen, eos = m.greedy_decode(prompt, 128)
    want, weos, want_logits = oracle_stream(ref, prompt, 128, cfg.max_seq)
    print(f"generated {len(got) - plen} tokens; smallest top-2 margin "
          f"{top2_margins(want_logits[plen - 1:]).min():.3e}")
    assert got.tolist() == want.tolist() and eos == weos
    st = m.stats()
    print(f"persistent={st['persistent']} grid={st['grid']} {st['gpu_ms']:.3f} ms for "
          f"{st['forwards']} forwards, {st['bytes_per_forward_mean'] / 1e6:.2f} MB/forward")
    assert st["persistent"]
    m.reset_cache()
    for pos in range(len(got) - 1):
        lg, am = m.eval_next_logits(int(got[pos]), pos)
        assert np.array_equal(lg, want_logits[pos]), \
            f"pos {pos}: max-abs {np.max(np.abs(lg - want_logits[pos]))}"
        assert am == int(np.argmax(want_logits[pos]))
    # the oracle's decoder state is the last forward of the same stream
    check_taps(m, ref, cfg)
    m.close()


def check_taps(m, ref, cfg):
    """sh_decode_tap of the last forward's last layer against the oracle's taps, bit for bit:
    x (layer output), q|k|v as projected (before QK-norm and RoPE), att, the SiLU gate and
    x2 (the residual after attention)."""
    Q, KV = cfg.qdim, cfg.kvdim
    qkv = m.tap(sh.SH_TAP_QKV)
    pairs = [("q", qkv[:Q], ref.tap(7, Q)), ("k", qkv[Q:Q + KV], ref.tap(8, KV)),
             ("v", qkv[Q + KV:], ref.tap(3, KV)),
             ("x", m.tap(sh.SH_TAP_X), ref.tap(0, cfg.dim)),
             ("att", m.tap(sh.SH_TAP_ATT), ref.tap(4, Q)),
             ("gate", m.tap(sh.SH_TAP_GATE), ref.tap(5, cfg.hidden)),
             ("x2", m.tap(sh.SH_TAP_X2), ref.tap(6, cfg.dim))]
    for name, got, want in pairs:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
            f"{name}: max-abs {np.max(np.abs(got - want))}"


def test_w8a8_taps_tiny(gpu):
    """The decode taps after each of several forwards of a tiny W8A8 model, bit for bit."""
    cfg = tiny_config()
    m, ref = build(cfg, seed=421, std=0.08, gains_seed=422)
    toks = sh.synth_tokens(12, 423, cfg.vocab)
    for pos, tok in enumerate(toks):
        got, _ = m.eval_next_logits(int(tok), pos)
        want = ref.forward_one(int(tok), pos)
        assert np.array_equal(got, want), f"pos {pos}"
        check_taps(m, ref, cfg)
    m.close()
