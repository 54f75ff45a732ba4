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


def build(cfg, seed, std=0.02, gains_seed=None, ref_kv=None):
    """The W8A8 model and the oracle's W8A8 decoder of the same weights (its cache type
    ref_kv, or the model's)."""
    w = sh.synth_weights(cfg, seed=seed, std=std)
    if gains_seed is not None:
        w = random_gains(w, gains_seed)
    m = sh.Model(cfg, sh.SH_DTYPE_W8A8)
    m.upload(w)
    print(m.describe())
    ref = oracle.Decoder(oracle.config_from(cfg, w8a8=True, kv_dtype=ref_kv),
                         w.rounded(sh.SH_DTYPE_W8A8), threads=THREADS)
    return m, ref


def check_steps(m, ref, tokens):
    """sh_decode_step against the oracle's forwardOne at every position: bit-identical logits
    (the W8A8 decode keeps the reference's float order wherever a value feeds a quantizer),
    which implies the 2e-2 bar, and the first-max argmax."""
    worst = 0.0
    for pos, tok in enumerate(tokens):
        got, am = m.eval_next_logits(int(tok), pos)
        want = ref.forward_one(int(tok), pos)
        err = float(np.max(np.abs(got - want)))
        worst = max(worst, err)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"pos {pos}: max-abs {err}"
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
    seed 1, 128 new tokens; identical token stream, the last forward's intermediates
    (sh_decode_tap, the counterpart of the engine's cache taps, engine_test.go:154-239)
    equal to the oracle's bit for bit both after the greedy decode (prompt cache from the
    full-sequence forward) and after a token-by-token replay, whose logits at all 143
    forwards are bit-identical to the oracle's."""
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
    # the decode's last forward, after the prompt's KV cache was filled by the full-sequence
    # forward: its intermediates equal the oracle's bit for bit
    check_taps(m, ref, cfg)
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


# ---- W8A8 beyond the batch-1 decode: int8 MFMA products (v_mfma_i32_16x16x64_i8) ----------

def fp16_exact(shape, seed, scale=1.0):
    """float32 values that fp16 holds exactly (so the operand planes carry them unchanged)."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape) * scale).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("shape", ["tiny", "stories110m"])
def test_w8a8_classifier_int8_product_bit_exact(gpu, shape):
    """The int8 MFMA product with its dequantization, through the classifier seam
    (sh_classifier_cf on a W8A8 model): every column of the channel-first input is quantized
    on its own (the bridge formula) and multiplied with the int8 classifier rows; the logits
    equal the oracle's or_mat_vec_w8a8 of that column bit for bit (exact int32 sums, then
    (float)acc * (s_w * s_a)). The inputs are values fp16 holds exactly, so the operand planes
    carry them unchanged into the quantizer. The device's int8 rows and scales are read
    back and equal the oracle's quantization of the fp32 rows."""
    cfg = tiny_config() if shape == "tiny" else sh.stories110m_config()
    w = sh.synth_weights(cfg, seed=431, std=0.05)
    m = sh.Model(cfg, sh.SH_DTYPE_W8A8)
    m.upload(w)
    cls = w.cls if w.cls is not None else w.embed
    q_want, s_want = oracle.quantize_rows(cls)
    assert np.array_equal(m.read_weights(-1, "cls"), q_want)
    assert np.array_equal(m.read_weights(-1, "cls.scale").view(np.uint32), s_want.view(np.uint32))
    S = 20 if shape == "tiny" else 72
    x = fp16_exact((cfg.dim, S), 432, 0.7)
    x[:, 3] = 0.0                         # an all-zero column: scale 1, every q = 0
    x[5, 4] = 1000.0                      # one large value: the rest quantize to small ints
    got = m.classifier_cf(x)
    for t in range(S):
        want = oracle.mat_vec_w8a8(q_want, s_want, x[:, t], THREADS)
        assert np.array_equal(got[:, t].view(np.uint32), want.view(np.uint32)), \
            f"column {t}: max-abs {np.max(np.abs(got[:, t] - want))}"
    m.close()


def check_w8a8_prefill(cfg, seed, std, gains_seed, S):
    """sh_prefill_logits (EvalLogits) of a W8A8 model against the oracle's W8A8 decoder at every
    position, bit for bit. The W8A8 forward keeps the decode's numerics wherever a value
    feeds a quantizer: fp32 operands, k and v rounded to the cache type, attention in the
    decode's float order, the decode's SiLU and final rmsNormVec; the int8 products are exact."""
    m, ref = build(cfg, seed=seed, std=std, gains_seed=gains_seed)
    toks = sh.synth_tokens(S, seed + 7, cfg.vocab)
    got = m.eval_logits(toks)
    assert got.shape == (cfg.vocab, S)
    for t in range(S):
        want = ref.forward_one(int(toks[t]), t)
        assert np.array_equal(got[:, t].view(np.uint32), want.view(np.uint32)), \
            f"position {t}: max-abs {np.max(np.abs(got[:, t] - want))}"
    print(f"W8A8 full-sequence logits, S={S}: bit-identical at every position")
    m.close()


def test_w8a8_prefill_logits_tiny(gpu):
    check_w8a8_prefill(tiny_config(), 441, 0.08, 442, 24)


def test_w8a8_prefill_logits_tiny_gqa_qknorm(gpu):
    check_w8a8_prefill(tiny_gqa_config(), 443, 0.08, 444, 17)


def test_w8a8_prefill_logits_stories110m(gpu):
    check_w8a8_prefill(sh.stories110m_config(), 0, 0.02, None, 64)


def test_w8a8_batch_decode_tiny(gpu):
    """Batched greedy decode of a W8A8 model (int8 MFMA products for the prompt forward and
    every step, B = 3 in lockstep): every row's token stream equals the oracle's W8A8 greedy
    decode of its prompt."""
    cfg = tiny_config(max_batch=4)
    m, ref = build(cfg, seed=451, std=0.08, gains_seed=452)
    prompts = sh.synth_tokens(3 * 10, 453, cfg.vocab).reshape(3, 10)
    got = m.batch_greedy_decode(prompts, 16)
    for b in range(3):
        ref.reset()
        want, _, margins = ref.greedy_decode(prompts[b], 16)
        print(f"row {b}: smallest top-2 margin {np.nanmin(margins):.3e}")
        assert got[b].tolist() == want.tolist(), f"row {b}"
    m.close()


def test_w8a8_batch_decode_gqa_bf16_kv(gpu):
    """The same with GQA, QK-norm and a bf16 KV cache (the attention reads the rounded cache)."""
    cfg = tiny_gqa_config(max_batch=2)
    m, ref = build(cfg, seed=455, std=0.08, gains_seed=456)
    prompts = sh.synth_tokens(2 * 13, 457, cfg.vocab).reshape(2, 13)
    got = m.batch_greedy_decode(prompts, 12)
    for b in range(2):
        ref.reset()
        want, _, _ = ref.greedy_decode(prompts[b], 12)
        assert got[b].tolist() == want.tolist(), f"row {b}"
    m.close()


def test_w8a8_window_decode_tiny(gpu):
    """Window decode of a W8A8 model (the full causal forward over the BOS-left-padded window
    at every step, decode.go:18-94): each step's token is the argmax of the oracle's W8A8
    decoder over the same window (its prompt pass), whose logits the window forward
    reproduces bit for bit."""
    cfg = tiny_config()
    m, ref = build(cfg, seed=461, std=0.08, gains_seed=462)
    seq = 12
    prompt = sh.synth_tokens(7, 463, cfg.vocab)
    got, plen, _ = m.window_greedy_decode(prompt, seq, 10)
    assert len(got) > plen
    hist = [int(t) for t in got[:plen]]
    for i in range(plen, len(got)):
        win = [1] * max(0, seq - len(hist)) + hist[-seq:]
        ref.reset()
        lg = ref.prompt_forward(win)
        assert int(got[i]) == int(np.argmax(lg)), f"step {i - plen}"
        hist.append(int(got[i]))
    m.close()
