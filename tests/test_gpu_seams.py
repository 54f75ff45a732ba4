"""GPU parity of the storiesane plugin seams and the stateless accelerators against the
oracle, through the C ABI: one layer over channel-first data (layerForward.run,
layer_other.go:27-37), the final RMSNorm and the classifier (offload.runRMSForward /
runClassifierForward, offload_other.go:22-27), matMulVocabSeqAccelerate (gemm_stub.go:5-7)
and forward.ConvEval (conv.go:11-52).

Bar: the float bar of the forward (max-abs 2e-2 on logits); the checks below are tighter
where the GPU keeps ~fp32 arithmetic (hidden states 1e-4 relative to their scale, the RMSNorm
1e-5), with the dtype-rounded weights on both sides. The seams compose: embedding -> layers ->
final norm -> classifier through them equals sh_prefill_logits.
"""
import os

import numpy as np
import pytest

import oracle
import stories_hip as sh
from helpers import random_gains, tiny_config, tiny_gqa_config

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))


def build(cfg, dtype, seed, std=0.05):
    w = random_gains(sh.synth_weights(cfg, seed=seed, std=std), seed + 1)
    m = sh.Model(cfg, dtype)
    m.upload(w)
    return m, oracle.config_from(cfg), w.rounded(dtype)


def embed_cf(w, toks):
    return np.ascontiguousarray(w.embed[np.asarray(toks)].T, np.float32)   # [D, S]


def rel_err(got, want):
    return float(np.max(np.abs(got - want))) / max(float(np.max(np.abs(want))), 1e-30)


@pytest.mark.parametrize("make_cfg,dtype,seq", [
    (lambda: tiny_config(residual_scale=0.5), sh.SH_DTYPE_F16, 24),
    (lambda: tiny_gqa_config(kv_dtype=sh.SH_KV_F32), sh.SH_DTYPE_BF16, 40),
])
def test_layer_forward_cf_matches_oracle(gpu, make_cfg, dtype, seq):
    cfg = make_cfg()
    m, ocfg, ow = build(cfg, dtype, 61)
    x = embed_cf(ow, sh.synth_tokens(seq, 62, cfg.vocab))
    for layer in range(cfg.n_layers):
        got = m.layer_forward_cf(layer, x)
        want = oracle.layer_forward_cf(ocfg, ow, layer, x, threads=THREADS)
        err = rel_err(got, want)
        print(f"layer {layer} S={seq}: rel {err:.2e}")
        assert got.shape == want.shape and err <= 1e-4, err
        x = want
    m.close()


@pytest.mark.parametrize("make_cfg,dtype,seq", [
    (lambda: tiny_config(residual_scale=0.5), sh.SH_DTYPE_F16, 24),
    (lambda: tiny_gqa_config(kv_dtype=sh.SH_KV_F32), sh.SH_DTYPE_BF16, 40),
    (lambda: sh.stories110m_config(), sh.SH_DTYPE_F16, 64),
])
def test_layer_taps_match_oracle(gpu, make_cfg, dtype, seq):
    """The layer's intermediates as the reference's fused layer programs return them
    (ane/mil/stories_dynamic.go:162: x2, q_rope, k_rope, v, att; :222: x_next, h1, h3), each
    block against the oracle's channel-first restatement of the same layer. The layer output
    equals sh_layer_forward_cf's bit for bit (the taps add work, they change none)."""
    cfg = make_cfg()
    std = 0.02 if cfg.dim == 768 else 0.05
    m, ocfg, ow = build(cfg, dtype, 67, std=std)
    x = embed_cf(ow, sh.synth_tokens(seq, 68, cfg.vocab))
    D, F, Q, KV = cfg.dim, cfg.hidden, cfg.qdim, cfg.kvdim
    names = [("x2", D), ("q_rope", Q), ("k_rope", KV), ("v", KV), ("att", Q)]
    for layer in range(min(cfg.n_layers, 2)):
        out, sdpa, ffn = m.layer_forward_cf_taps(layer, x)
        np.testing.assert_array_equal(out, m.layer_forward_cf(layer, x))
        w_out, w_sdpa, w_ffn = oracle.layer_forward_cf_taps(ocfg, ow, layer, x, threads=THREADS)
        assert sdpa.shape == w_sdpa.shape and ffn.shape == w_ffn.shape
        np.testing.assert_array_equal(ffn[:D], out)
        o = 0
        for name, n in names:
            err = rel_err(sdpa[o:o + n], w_sdpa[o:o + n])
            print(f"layer {layer} sdpa {name}: rel {err:.2e}")
            assert err <= 1e-4, (name, err)
            o += n
        for name, a, b in (("x_next", 0, D), ("h1", D, D + F), ("h3", D + F, D + 2 * F)):
            err = rel_err(ffn[a:b], w_ffn[a:b])
            print(f"layer {layer} ffn {name}: rel {err:.2e}")
            assert err <= 1e-4, (name, err)
        x = w_out
    m.close()


def test_one_layer_model_is_a_compiled_layer(gpu):
    # compileStoriesLayerForwardFunc's counterpart: a model holding one layer and no globals
    cfg = tiny_config(residual_scale=0.5)
    m, ocfg, ow = build(cfg, sh.SH_DTYPE_F16, 65)
    x = embed_cf(ow, sh.synth_tokens(21, 66, cfg.vocab))
    one = tiny_config(residual_scale=0.5, n_layers=1)
    lm = sh.Model(one, sh.SH_DTYPE_F16)
    src = sh.synth_weights(cfg, seed=65, std=0.05)
    src = random_gains(src, 66)
    lw = src.layers[1]
    lm._upload_layer(0, lw)
    with pytest.raises(sh.ShError, match="not fully uploaded"):
        lm.rms_final_cf(x)
    np.testing.assert_array_equal(lm.layer_forward_cf(0, x), m.layer_forward_cf(1, x))
    lm.close()
    m.close()


def test_rms_final_and_classifier_cf_match_oracle(gpu):
    cfg = tiny_config()
    m, ocfg, ow = build(cfg, sh.SH_DTYPE_F16, 71)
    x = np.random.default_rng(72).standard_normal((cfg.dim, 33)).astype(np.float32)
    got = m.rms_final_cf(x)
    want = oracle.rms_norm_final_cf(x, ow.rms_final, cfg.norm_eps)
    assert rel_err(got, want) <= 1e-5
    logits = m.classifier_cf(want)
    cls = ow.embed if ow.cls is None else ow.cls
    ref = oracle.matmul_vocab_seq(cls, want, threads=THREADS)
    assert logits.shape == (cfg.vocab, 33) and rel_err(logits, ref) <= 1e-4
    m.close()


def test_seams_compose_to_eval_logits(gpu):
    cfg = tiny_config(residual_scale=0.5)
    m, ocfg, ow = build(cfg, sh.SH_DTYPE_F16, 81)
    toks = sh.synth_tokens(29, 82, cfg.vocab)
    x = embed_cf(ow, toks)
    for layer in range(cfg.n_layers):
        x = m.layer_forward_cf(layer, x)
    logits = m.classifier_cf(m.rms_final_cf(x))
    full = m.eval_logits(toks)
    # the seams carry the activations into their products as hi/lo fp16 pairs, EvalLogits
    # (fp16) as one fp16 plane: the two agree to the plane's rounding, both within the bar
    assert float(np.max(np.abs(logits - full))) <= 2e-3
    want = oracle.eval_logits_cf(ocfg, ow, toks, threads=THREADS)
    assert float(np.max(np.abs(logits - want))) <= 2e-2
    assert float(np.max(np.abs(full - want))) <= 2e-2
    m.close()


def test_seam_argument_errors(gpu):
    cfg = tiny_config()
    m, _, _ = build(cfg, sh.SH_DTYPE_F16, 91)
    x = np.zeros((cfg.dim, 4), np.float32)
    with pytest.raises(sh.ShError, match="layer out of range"):
        m.layer_forward_cf(cfg.n_layers, x)
    with pytest.raises(sh.ShError, match="bad arguments"):
        m.layer_forward_cf(0, np.zeros((cfg.dim, cfg.max_seq + 1), np.float32))
    m.close()


@pytest.mark.parametrize("vocab,dim,seq", [(512, 128, 7), (32000, 768, 64)])
def test_matmul_vocab_seq_matches_oracle(gpu, vocab, dim, seq):
    rng = np.random.default_rng(vocab + seq)
    embed = (0.02 * rng.standard_normal((vocab, dim))).astype(np.float32)
    x = rng.standard_normal((dim, seq)).astype(np.float32)
    got = sh.matmul_vocab_seq(embed, x)
    # the device rounds embed to fp16 once: bit-level agreement target is the oracle on the
    # rounded embedding, the reference's fp32 product within the float bar
    e16 = sh.round_dtype(embed, sh.SH_DTYPE_F16)
    assert rel_err(got, oracle.matmul_vocab_seq(e16, x, threads=THREADS)) <= 1e-5
    assert float(np.max(np.abs(got - oracle.matmul_vocab_seq(embed, x, threads=THREADS)))) <= 2e-2


def test_conv_eval_matches_linear_cf(gpu):
    rng = np.random.default_rng(5)
    out_dim, in_dim, s = 192, 96, 37
    w = (0.1 * rng.standard_normal((out_dim, in_dim))).astype(np.float32)
    x = rng.standard_normal((s, in_dim)).astype(np.float32)
    conv = sh.Conv(w)
    got = conv.eval(x)
    # ConvEval: transpose to [in, s], the 1x1 conv (linearCF), transpose back
    want = oracle.linear_cf(sh.round_dtype(w, sh.SH_DTYPE_F16), np.ascontiguousarray(x.T)).T
    assert got.shape == (s, out_dim) and rel_err(got, want) <= 1e-5
    np.testing.assert_array_equal(conv.eval(x), got)   # a compiled kernel is reusable
    conv.close()
