"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

The reference ships no golden vectors for this path, so each oracle function is pinned by
the reference's own known-answer tests where they exist (EmbedLookup, fillDecodeWindow),
by closed forms and invariants, by library routines (numpy float16 casts, torch bfloat16
casts, torch rms_norm / silu / scaled_dot_product_attention), and by a float64 brute-force
forward on tiny shapes. Each check is chosen so a plausible slip (a dropped gain, a swapped
RoPE sign, a transposed operand, the wrong KV head, a missing residual scale) fails it.
"""
import math

import numpy as np
import pytest
import scipy.special
import torch

import oracle
import stories_hip as sh
from helpers import deepnet_alpha, random_gains, tiny_config, tiny_gqa_config, torch_forward_f64

L = oracle.load()


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- dtype rounding ----------------------------------------------------------------------

def test_half_round_matches_numpy_float16():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 5, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, -65520.0, 6.0e-8, 2.9e-8, 3.0e-8,
                  6.1035156e-05, 6.097555e-05, 1.0009766, 1.00048828125, 1.00146484375],
                 np.float32),
    ])
    got = np.array([L.or_half_round(float(v)) for v in vals], np.float32)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
                           np.array([1.00390625, 1.01171875, -3.0e38, 1.0e-40], np.float32)])
    got = np.array([L.or_bf16_round(float(v)) for v in vals], np.float32)
    want = torch.tensor(vals).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


# ---- scalar building blocks ---------------------------------------------------------------

def test_rms_norm_closed_form_and_gain():
    rng = np.random.default_rng(2)
    x = f32(rng.standard_normal(768) * 3)
    ones = np.ones(768, np.float32)
    out = np.empty(768, np.float32)
    L.or_rms_norm_vec(oracle.fp(out), oracle.fp(x), oracle.fp(ones), 768, 1e-5)
    ms = float(np.mean(x.astype(np.float64) ** 2))
    # RMS(out) = 1/sqrt(1 + eps/mean(x^2)) for unit gain
    assert abs(math.sqrt(np.mean(out.astype(np.float64) ** 2)) - 1 / math.sqrt(1 + 1e-5 / ms)) < 1e-6
    g = f32(0.5 + rng.random(768))
    out2 = np.empty(768, np.float32)
    L.or_rms_norm_vec(oracle.fp(out2), oracle.fp(x), oracle.fp(g), 768, 1e-5)
    want = torch.nn.functional.rms_norm(torch.tensor(x, dtype=torch.float64), (768,),
                                        torch.tensor(g, dtype=torch.float64), eps=1e-5).numpy()
    np.testing.assert_allclose(out2, want, rtol=2e-7, atol=1e-7)


def test_mat_vec_against_float64_product_and_threads():
    rng = np.random.default_rng(3)
    W = f32(rng.standard_normal((300, 77)))
    v = f32(rng.standard_normal(77))
    out1 = np.empty(300, np.float32)
    out4 = np.empty(300, np.float32)
    L.or_mat_vec(oracle.fp(out1), oracle.fp(W), oracle.fp(v), 300, 77, 1)
    L.or_mat_vec(oracle.fp(out4), oracle.fp(W), oracle.fp(v), 300, 77, 4)
    want = W.astype(np.float64) @ v.astype(np.float64)
    np.testing.assert_allclose(out1, want, rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(out1, out4)  # threads change scheduling, not sums
    # matVec keeps the reference's sequential float32 order: row 0 recomputed in order
    s = np.float32(0)
    for c in range(77):
        s = np.float32(s + np.float32(W[0, c] * v[c]))
    assert out1[0] == s


def test_silu_and_softmax_and_argmax():
    xs = np.linspace(-30, 30, 601).astype(np.float32)
    got = np.array([L.or_silu(float(x)) for x in xs], np.float32)
    want = xs.astype(np.float64) * scipy.special.expit(xs.astype(np.float64))
    np.testing.assert_allclose(got, want, rtol=3e-7, atol=1e-30)

    rng = np.random.default_rng(4)
    s = f32(rng.standard_normal(143) * 4)
    p = np.empty(143, np.float32)
    L.or_softmax_prefix(oracle.fp(p), oracle.fp(s), 143)
    np.testing.assert_allclose(p, scipy.special.softmax(s.astype(np.float64)), rtol=1e-6, atol=1e-9)
    assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-6
    p1 = np.empty(1, np.float32)
    L.or_softmax_prefix(oracle.fp(p1), oracle.fp(f32([7.5])), 1)
    assert p1[0] == 1.0  # one key: probability exactly 1

    v = f32([0.5, 2.0, -1.0, 2.0, 1.9])
    assert L.or_argmax(oracle.fp(v), 5) == 1  # first maximum (infer.go:373-383)


def test_rope_tables():
    hd, S = 64, 256
    c = np.empty(S * hd // 2, np.float32)
    s = np.empty(S * hd // 2, np.float32)
    L.or_rope_tables(oracle.fp(c), oracle.fp(s), S, hd, 10000.0)
    c = c.reshape(S, hd // 2)
    s = s.reshape(S, hd // 2)
    assert np.all(c[0] == 1) and np.all(s[0] == 0)  # position 0 is the identity
    ang = np.arange(S)[:, None] * (10000.0 ** (-np.arange(0, hd, 2) / hd))[None, :]
    np.testing.assert_allclose(c, np.cos(ang), atol=6e-8)
    np.testing.assert_allclose(s, np.sin(ang), atol=6e-8)


# ---- quantizer (bridge/ane_bridge.m:374-399) --------------------------------------------

def test_quantize_known_answers():
    # scale = 1/127; 1 -> 127, -0.5 -> -63.5 -> half away -> -64, 0.25 -> 31.75 -> 32
    q, s = oracle.quantize_tensor(f32([1.0, -0.5, 0.25, 0.0, 0.0039]))
    assert s == np.float32(1.0) / np.float32(127.0)
    assert q.tolist() == [127, -64, 32, 0, 0]
    # all zeros: scale 0 -> 1, values 0
    q, s = oracle.quantize_tensor(np.zeros(5, np.float32))
    assert s == 1.0 and q.tolist() == [0] * 5
    # exact half steps round away from zero: x/scale = +-k.5
    scale = np.float32(2.0) / np.float32(127.0)
    x = f32([2.0, 0.5 * scale, -0.5 * scale, 1.5 * scale, -2.5 * scale])
    q, s = oracle.quantize_tensor(x)
    assert s == scale
    xs = (x / s).astype(np.float32)
    want = [int(np.trunc(np.float32(v + (np.float32(0.5) if v >= 0 else np.float32(-0.5))))) for v in xs]
    assert q.tolist() == want
    assert q.tolist()[0] == 127
    # per-row with one row is the bridge's per-tensor formula
    rng = np.random.default_rng(5)
    a = f32(rng.standard_normal(999))
    qt, st = oracle.quantize_tensor(a)
    qr, sr = oracle.quantize_rows(a.reshape(1, -1))
    np.testing.assert_array_equal(qt, qr.reshape(-1))
    assert st == sr[0]


def test_quantize_rows_dequantize_error_bound():
    rng = np.random.default_rng(6)
    w = f32(rng.standard_normal((64, 128)) * 0.02)
    w[3] = 0.0
    q, s = oracle.quantize_rows(w)
    assert s[3] == 1.0 and np.all(q[3] == 0)
    want_s = np.abs(w).max(axis=1) / np.float32(127)
    want_s[want_s == 0] = 1.0
    np.testing.assert_array_equal(s, want_s)
    dq = oracle.dequantize_rows(q, s)
    np.testing.assert_array_equal(dq, q.astype(np.float32) * s[:, None])
    assert np.all(np.abs(dq - w) <= s[:, None] * 0.5 + 1e-9)  # half a step at most
    assert q.max() <= 127 and q.min() >= -128


def test_mat_vec_w8a8_exact_integer_path():
    rng = np.random.default_rng(7)
    w = f32(rng.standard_normal((96, 64)))
    x = f32(rng.standard_normal(64))
    qw, sw = oracle.quantize_rows(w)
    qa, sa = oracle.quantize_tensor(x)
    out = np.empty(96, np.float32)
    L.or_mat_vec_w8a8(oracle.fp(out), qw.ctypes.data_as(oracle.C.POINTER(oracle.C.c_int8)), oracle.fp(sw),
                      oracle.fp(x), 96, 64, 1)
    acc = qw.astype(np.int64) @ qa.astype(np.int64)
    want = acc.astype(np.float32) * (sw * sa)
    np.testing.assert_array_equal(out, want)
    np.testing.assert_allclose(out, w.astype(np.float64) @ x, atol=0.4)  # int8 rounding error


# ---- reference known-answer tests ---------------------------------------------------------

def test_embed_lookup_cf_known_answers():
    # ane/stories/cpu_test.go:33-52 and :56-74
    dim, seq, vocab = 3, 2, 5
    embed = f32(np.arange(1, vocab * dim + 1))
    out = np.empty(dim * seq, np.float32)
    toks = np.array([1, 3], np.uint16)
    L.or_embed_lookup_cf(oracle.fp(out), oracle.fp(embed), vocab, toks.ctypes.data_as(oracle.C.POINTER(oracle.C.c_uint16)), dim, seq)
    assert out[0] == embed[1 * dim + 0] and out[1] == embed[3 * dim + 0]
    embed2 = f32([1, 2, 3, 4, 5, 6])
    toks2 = np.array([1, 5], np.uint16)  # 5 is out of range for vocab 2
    L.or_embed_lookup_cf(oracle.fp(out), oracle.fp(embed2), 2, toks2.ctypes.data_as(oracle.C.POINTER(oracle.C.c_uint16)), dim, seq)
    for d in range(dim):
        assert out[d * seq + 0] == embed2[dim + d]
        assert out[d * seq + 1] == 0


def test_fill_decode_window_known_answer():
    # ane/storiesane/engine_test.go:313-322
    dst = np.zeros(5, np.uint16)
    toks = np.array([7, 8], np.int32)
    L.or_fill_decode_window(dst.ctypes.data_as(oracle.C.POINTER(oracle.C.c_uint16)), 5,
                            toks.ctypes.data_as(oracle.C.POINTER(oracle.C.c_int32)), 2)
    assert dst.tolist() == [1, 1, 1, 7, 8]
    long = np.arange(10, 20, dtype=np.int32)
    L.or_fill_decode_window(dst.ctypes.data_as(oracle.C.POINTER(oracle.C.c_uint16)), 5,
                            long.ctypes.data_as(oracle.C.POINTER(oracle.C.c_int32)), 10)
    assert dst.tolist() == [15, 16, 17, 18, 19]


# ---- whole-forward pins --------------------------------------------------------------------

@pytest.mark.parametrize("gqa", [False, True])
def test_decoder_matches_float64_forward(gqa):
    cfg = tiny_gqa_config(kv_dtype=sh.SH_KV_F32) if gqa else tiny_config()
    w = random_gains(sh.synth_weights(cfg, seed=11, std=0.08), 12)
    toks = sh.synth_tokens(20, 13, cfg.vocab)
    ref = torch_forward_f64(cfg, w, toks)
    dec = oracle.Decoder(oracle.config_from(cfg), w)
    for t, tok in enumerate(toks):
        got = dec.forward_one(int(tok), t)
        np.testing.assert_allclose(got, ref[t], atol=2e-5, rtol=0)


def test_decoder_residual_scale_matches_float64_forward():
    cfg = tiny_config(residual_scale=deepnet_alpha(2))
    w = sh.synth_weights(cfg, seed=21, std=0.1)
    toks = sh.synth_tokens(10, 22, cfg.vocab)
    ref = torch_forward_f64(cfg, w, toks)
    dec = oracle.Decoder(oracle.config_from(cfg), w)
    for t, tok in enumerate(toks):
        np.testing.assert_allclose(dec.forward_one(int(tok), t), ref[t], atol=2e-5, rtol=0)


@pytest.mark.parametrize("alpha,layers", [(1.0, 2), (None, 2), (None, 3)])
def test_eval_logits_cf_matches_float64_forward(alpha, layers):
    cfg = tiny_config(n_layers=layers,
                      residual_scale=deepnet_alpha(layers) if alpha is None else alpha)
    w = random_gains(sh.synth_weights(cfg, seed=31, std=0.08), 32)
    toks = sh.synth_tokens(24, 33, cfg.vocab)
    got = oracle.eval_logits_cf(oracle.config_from(cfg), w, toks, threads=2)
    ref = torch_forward_f64(cfg, w, toks)
    np.testing.assert_allclose(got.T, ref, atol=2e-5, rtol=0)


def test_eval_logits_is_causal_and_zeroes_out_of_range_tokens():
    cfg = tiny_config()
    w = sh.synth_weights(cfg, seed=41, std=0.08)
    toks = sh.synth_tokens(12, 42, cfg.vocab).astype(np.int64)
    a = oracle.eval_logits_cf(oracle.config_from(cfg), w, toks)
    toks2 = toks.copy()
    toks2[7] = (toks2[7] + 1) % cfg.vocab
    b = oracle.eval_logits_cf(oracle.config_from(cfg), w, toks2)
    np.testing.assert_array_equal(a[:, :7], b[:, :7])  # masked scores give exactly 0 weight
    assert not np.array_equal(a[:, 7], b[:, 7])
    # an out-of-range id is a zero embedding column (cpu.go:41-72): same as a zero row
    free = next(v for v in range(cfg.vocab) if v not in set(toks.tolist()))
    toks3 = toks.copy()
    toks3[0] = cfg.vocab + 5
    c = oracle.eval_logits_cf(oracle.config_from(cfg), w, toks3)
    w0 = sh.Weights(w.layers, w.embed.copy(), w.rms_final, w.embed.copy())
    w0.embed[free] = 0
    toks4 = toks.copy()
    toks4[0] = free
    d = oracle.eval_logits_cf(oracle.config_from(cfg), w0, toks4)
    np.testing.assert_allclose(c, d, atol=1e-6)


def test_decoder_closed_forms():
    cfg = tiny_config(n_layers=2)
    w = sh.synth_weights(cfg, seed=51, std=0.08)
    # zero projections: the residual stream is the embedding, logits = E . rmsnorm(E[tok])
    for lw in w.layers:
        for k in sh.LAYER_KEYS:
            lw[k] = np.zeros_like(lw[k])
    dec = oracle.Decoder(oracle.config_from(cfg), w)
    tok = 77
    got = dec.forward_one(tok, 0)
    e = w.embed[tok].astype(np.float64)
    xn = e / np.sqrt(np.mean(e * e) + 1e-5)
    np.testing.assert_allclose(got, w.embed.astype(np.float64) @ xn, atol=1e-5)
    # all-zero model: logits 0, argmax 0
    for lw in w.layers:
        pass
    wz = sh.Weights(w.layers, np.zeros_like(w.embed), w.rms_final, None)
    decz = oracle.Decoder(oracle.config_from(cfg), wz)
    assert np.all(decz.forward_one(5, 0) == 0)
    toks, eos, _ = decz.greedy_decode([5, 6], 3)
    assert toks.tolist() == [5, 6, 0, 0, 0] and not eos


def test_attention_at_position_zero_is_v():
    cfg = tiny_config(n_layers=1)
    w = sh.synth_weights(cfg, seed=61, std=0.08)
    dec = oracle.Decoder(oracle.config_from(cfg), w)
    dec.forward_one(9, 0)
    np.testing.assert_array_equal(dec.tap(4, cfg.qdim), dec.tap(3, cfg.kvdim))


def test_greedy_decode_bookkeeping():
    cfg = tiny_config(n_layers=1, max_seq=16)
    w = sh.synth_weights(cfg, seed=71, std=0.08)
    dec = oracle.Decoder(oracle.config_from(cfg), w)
    # maxSeq stop (infer.go:179): 13-token prompt leaves room for 3
    p = sh.synth_tokens(13, 72, cfg.vocab)
    toks, eos, _ = dec.greedy_decode(p, 10)
    assert len(toks) == 16 and toks[:13].tolist() == p.tolist()
    # the generated ids are the argmax of each step's logits
    dec2 = oracle.Decoder(oracle.config_from(cfg), w)
    for pos in range(12):
        dec2.forward_one(int(p[pos]), pos)
    nxt = int(np.argmax(dec2.forward_one(int(p[12]), 12)))
    assert toks[13] == nxt
    # an over-long prompt keeps its last max_seq ids; no room -> no new tokens
    p2 = sh.synth_tokens(20, 73, cfg.vocab)
    toks2, _, _ = dec.greedy_decode(p2, 4)
    assert toks2.tolist() == p2[-16:].tolist()
    # empty prompt -> [BOS]
    toks3, _, _ = dec.greedy_decode([], 2)
    assert toks3[0] == 1 and len(toks3) == 3
    # out-of-range prompt id is an error
    with pytest.raises(ValueError):
        dec.greedy_decode([cfg.vocab], 2)
    # EOS stop: every step's argmax is EOS=2 (zero projections, constant embedding,
    # classifier row 2 = ones)
    for lw in w.layers:
        for k in sh.LAYER_KEYS:
            lw[k] = np.zeros_like(lw[k])
    emb = np.full_like(w.embed, 0.01)
    cls = np.zeros_like(w.embed)
    cls[2] = 1.0
    dec3 = oracle.Decoder(oracle.config_from(cfg), sh.Weights(w.layers, emb, w.rms_final, cls))
    toks4, eos4, _ = dec3.greedy_decode([5, 9], 10)
    assert eos4 and toks4.tolist() == [5, 9, 2]


def test_kv_cache_decode_equals_causal_prefill():
    """Decode step t equals column t of the full-sequence forward (alpha 1): ties the
    KV-cache decoder (infer.go) to the channel-first forward (engine.go:804-842)."""
    cfg = tiny_gqa_config(kv_dtype=sh.SH_KV_F32)
    w = random_gains(sh.synth_weights(cfg, seed=81, std=0.08), 82)
    toks = sh.synth_tokens(16, 83, cfg.vocab)
    cf = oracle.eval_logits_cf(oracle.config_from(cfg), w, toks)
    dec = oracle.Decoder(oracle.config_from(cfg), w)
    for t, tok in enumerate(toks):
        np.testing.assert_allclose(dec.forward_one(int(tok), t), cf[:, t], atol=1e-5)


@pytest.mark.parametrize("gqa,w8a8,kv", [(False, False, sh.SH_KV_F32), (True, False, sh.SH_KV_BF16),
                                         (False, True, sh.SH_KV_F16), (True, True, sh.SH_KV_F32)])
def test_prompt_pass_equals_forward_one_bitwise(gqa, w8a8, kv):
    """The layer-major prompt pass (or_prompt_forward, which the oracle's greedy decode uses
    for the prompt) against forwardOne called per position: the same logits and the same
    K/V cache, bit for bit, so the next forwardOne after either gives identical logits. An
    odd hidden size leaves a partial four-row group, 27 tokens a partial eight-token block,
    and a second pass starting at position 27 checks pos0 > 0."""
    mk = tiny_gqa_config if gqa else tiny_config
    cfg = mk(kv_dtype=kv, hidden=250)
    w = random_gains(sh.synth_weights(cfg, seed=84, std=0.08), 85)
    oc = oracle.config_from(cfg, w8a8=w8a8)
    toks = sh.synth_tokens(40, 86, cfg.vocab)
    one, turned = oracle.Decoder(oc, w, threads=3), oracle.Decoder(oc, w, threads=2)
    for t in range(27):
        a = one.forward_one(int(toks[t]), t)
    b = turned.prompt_forward(toks[:27])
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for t in range(27, 39):
        a = one.forward_one(int(toks[t]), t)
    b = turned.prompt_forward(toks[27:39], pos0=27)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    a, b = one.forward_one(int(toks[39]), 39), turned.forward_one(int(toks[39]), 39)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    with pytest.raises(ValueError):
        turned.prompt_forward(toks[:30], pos0=cfg.max_seq - 29)
    one.close()
    turned.close()


@pytest.mark.parametrize("gqa,w8a8", [(False, False), (True, True)])
def test_prompt_pass_logits_range_equals_forward_one_bitwise(gqa, w8a8):
    """or_prompt_forward_logits (a teacher-forced pass over a given stream keeping the logits
    from one position on, used to check the batched decode at every step) against forwardOne
    per position: every kept row bit-identical, 21 rows leaving a partial eight-token block of
    the classifier product."""
    mk = tiny_gqa_config if gqa else tiny_config
    cfg = mk()
    w = random_gains(sh.synth_weights(cfg, seed=87, std=0.08), 88)
    oc = oracle.config_from(cfg, w8a8=w8a8)
    toks = sh.synth_tokens(33, 89, cfg.vocab)
    one, turned = oracle.Decoder(oc, w, threads=3), oracle.Decoder(oc, w, threads=2)
    want = np.stack([one.forward_one(int(toks[t]), t) for t in range(33)])
    got = turned.prompt_forward_logits(toks, first=12)
    assert got.shape == (21, cfg.vocab)
    assert np.array_equal(got.view(np.uint32), want[12:].view(np.uint32))
    with pytest.raises(ValueError):
        turned.prompt_forward_logits(toks, first=33)
    one.close()
    turned.close()


def test_w8a8_decoder_tracks_fp32():
    cfg = tiny_config()
    w = sh.synth_weights(cfg, seed=91, std=0.08)
    toks = sh.synth_tokens(8, 92, cfg.vocab)
    ref = oracle.Decoder(oracle.config_from(cfg), w)
    q = oracle.Decoder(oracle.config_from(cfg, w8a8=True), w)
    for t, tok in enumerate(toks):
        a = ref.forward_one(int(tok), t)
        b = q.forward_one(int(tok), t)
        assert np.max(np.abs(a - b)) < 0.05 * np.max(np.abs(a)) + 0.02
        assert not np.array_equal(a, b)


def test_kv_storage_rounding():
    cfg = tiny_config(n_layers=1)
    w = sh.synth_weights(cfg, seed=95, std=0.08)
    d32 = oracle.Decoder(oracle.config_from(cfg, kv_dtype=oracle.OR_KV_F32), w)
    d16 = oracle.Decoder(oracle.config_from(cfg, kv_dtype=oracle.OR_KV_F16), w)
    for t in range(4):
        a = d32.forward_one(t + 3, t)
        b = d16.forward_one(t + 3, t)
    assert 0 < np.max(np.abs(a - b)) < 1e-2


# ---- seam pieces: the channel-first forward factored as the plugin seams use it ------------

def test_seam_pieces_compose_to_eval_logits_exactly():
    cfg = tiny_config(n_layers=3, residual_scale=deepnet_alpha(3))
    w = random_gains(sh.synth_weights(cfg, seed=101, std=0.08), 102)
    toks = sh.synth_tokens(19, 103, cfg.vocab)
    ocfg = oracle.config_from(cfg)
    x = np.ascontiguousarray(w.embed[toks].T)
    for layer in range(cfg.n_layers):
        x = oracle.layer_forward_cf(ocfg, w, layer, x, threads=2)
    xn = oracle.rms_norm_final_cf(x, w.rms_final, cfg.norm_eps)
    logits = oracle.matmul_vocab_seq(w.embed, xn, threads=2)
    np.testing.assert_array_equal(logits, oracle.eval_logits_cf(ocfg, w, toks, threads=2))


def test_linear_vocab_matmul_and_final_norm_against_float64():
    rng = np.random.default_rng(104)
    wt = rng.standard_normal((48, 80)).astype(np.float32)
    x = rng.standard_normal((80, 13)).astype(np.float32)
    ref = wt.astype(np.float64) @ x.astype(np.float64)
    np.testing.assert_allclose(oracle.linear_cf(wt, x), ref, atol=1e-4, rtol=0)
    np.testing.assert_allclose(oracle.matmul_vocab_seq(wt, x), ref, atol=1e-4, rtol=0)
    # an operand transposed or an index swapped would fail the non-square case above; the
    # final RMSNorm (cpu.go:97-111) against its float64 closed form, with non-unit gains
    g = (0.5 + rng.random(80)).astype(np.float32)
    got = oracle.rms_norm_final_cf(x, g, 1e-5)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd ** 2).mean(axis=0, keepdims=True) + 1e-5) * g[:, None]
    np.testing.assert_allclose(got, want, atol=1e-6, rtol=1e-6)


def test_splitmix64_draws_known_answers():
    """The test helper's splitmix64 against the generator's published outputs for seed 0."""
    from helpers import splitmix64_uniforms
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    got = splitmix64_uniforms(0, 4)
    assert [int(u * 9007199254740992.0) for u in got] == [w >> 11 for w in want]


def test_sample_from_logits_is_inverse_cdf_of_softmax():
    """or_sample_from_logits (infer.go:347-371) against the mathematics: the argmax rule at
    temperature <= 1e-6 (first maximum); otherwise the index i with cdf[i-1] < u <= cdf[i] for
    the softmax of logits/T (scipy, float64), with the reported slack its distance from those
    bounds; closed forms on two equal logits; the draw's end points."""
    from scipy.special import softmax
    lg = np.array([0.5, 2.0, 2.0, -1.0], np.float32)
    assert oracle.sample_from_logits(lg, 0.0, 0.9) == (1, 0.0)
    assert oracle.sample_from_logits(lg, 1e-7, 0.1)[0] == 1
    two = np.zeros(2, np.float32)
    assert oracle.sample_from_logits(two, 1.0, 0.25) == (0, 0.25)
    assert oracle.sample_from_logits(two, 1.0, 0.75) == (1, 0.25)
    assert oracle.sample_from_logits(two, 1.0, 0.0)[0] == 0
    rng = np.random.default_rng(91)
    for temp in (0.8, 0.5, 1.7):
        lg = (rng.standard_normal(300) * 1.5).astype(np.float32)
        inv_t = float(np.float32(1.0) / np.float32(temp))
        cdf = np.cumsum(softmax(lg.astype(np.float64) * inv_t))
        for u in rng.random(400):
            i, slack = oracle.sample_from_logits(lg, temp, float(u))
            lo = cdf[i - 1] if i else 0.0
            assert lo - 1e-12 <= u <= cdf[i] + 1e-12, (temp, u, i)
            assert slack == pytest.approx(min(u - lo, cdf[i] - u), abs=1e-12)
        assert oracle.sample_from_logits(lg, temp, 0.0)[0] == 0   # target 0: the first index


def test_eval_logits_reference_threading_same_values():
    """The forward timed with the reference's threading (linearCF and attention serial) gives
    the same logits, bit for bit, as the threaded one (each output's sum keeps its order)."""
    cfg = tiny_gqa_config(qk_norm=1)
    w = random_gains(sh.synth_weights(cfg, seed=92, std=0.08), 93)
    oc = oracle.config_from(cfg)
    toks = sh.synth_tokens(21, 94, cfg.vocab)
    a = oracle.eval_logits_cf(oc, w, toks, threads=4)
    b = oracle.eval_logits_cf(oc, w, toks, threads=3, reference_threading=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
