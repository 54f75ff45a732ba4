"""GPU parity of the batch-1 decode path against the CPU oracle, through the C ABI.

Bars (stated per test): logits within max-abs 2e-2 of the fp32 oracle fed the same
dtype-rounded weights, greedy token streams identical, int8 quantize/dequantize bit-exact.
"""
import os

import numpy as np
import pytest

import oracle
import stories_hip as sh
from helpers import oracle_stream, random_gains, tiny_config, tiny_gqa_config, top2_margins

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2  # max-abs logits bar
THREADS = max(1, min(16, os.cpu_count() or 1))


def build(cfg, dtype, seed, std=0.02, gains_seed=None):
    w = sh.synth_weights(cfg, seed=seed, std=std)
    if gains_seed is not None:
        w = random_gains(w, gains_seed)
    m = sh.Model(cfg, dtype)
    m.upload(w)
    print(m.describe())
    ref = oracle.Decoder(oracle.config_from(cfg, w8a8=(dtype == sh.SH_DTYPE_W8A8)),
                         w.rounded(dtype), threads=THREADS)
    return m, ref, w


def check_steps(m, ref, tokens, tol=LOGIT_TOL):
    worst = 0.0
    for pos, tok in enumerate(tokens):
        got, am = m.eval_next_logits(int(tok), pos)
        want = ref.forward_one(int(tok), pos)
        err = float(np.max(np.abs(got - want)))
        worst = max(worst, err)
        assert err <= tol, f"pos {pos}: max-abs {err}"
        assert am == int(np.argmax(got))
        assert am == int(np.argmax(want)), f"pos {pos}: argmax {am} vs {np.argmax(want)}"
    print(f"max-abs logits error over {len(tokens)} positions: {worst:.3e}")
    return worst


@pytest.mark.parametrize("dtype,kv", [(sh.SH_DTYPE_F16, sh.SH_KV_F32), (sh.SH_DTYPE_F16, sh.SH_KV_F16),
                                      (sh.SH_DTYPE_BF16, sh.SH_KV_BF16)])
def test_decode_step_tiny(gpu, dtype, kv):
    cfg = tiny_config(kv_dtype=kv)
    m, ref, _ = build(cfg, dtype, seed=101, std=0.08, gains_seed=102)
    toks = sh.synth_tokens(40, 103, cfg.vocab)
    worst = check_steps(m, ref, toks)
    assert worst < 1e-3
    m.close()


def test_decode_step_graph_path_shape(gpu):
    """A shape without a persistent-kernel instantiation runs the per-stage graph path."""
    cfg = tiny_config(dim=256, hidden=512, n_heads=8, n_kv_heads=4, head_dim=32)
    m, ref, _ = build(cfg, sh.SH_DTYPE_F16, seed=105, std=0.06, gains_seed=106)
    assert check_steps(m, ref, sh.synth_tokens(24, 107, cfg.vocab)) < 1e-3
    p = sh.synth_tokens(6, 108, cfg.vocab)
    got, _, _ = m.greedy_decode(p, 20)
    want, _, _ = ref.greedy_decode(p, 20)
    assert got.tolist() == want.tolist()
    assert not m.stats()["persistent"]
    m.close()


def test_decode_step_tiny_gqa_qknorm(gpu):
    cfg = tiny_gqa_config()
    m, ref, _ = build(cfg, sh.SH_DTYPE_BF16, seed=111, std=0.08, gains_seed=112)
    toks = sh.synth_tokens(48, 113, cfg.vocab)
    assert check_steps(m, ref, toks) < 1e-3
    m.close()


def test_decode_step_tiny_residual_scale(gpu):
    cfg = tiny_config(residual_scale=0.5, n_layers=3)
    m, ref, _ = build(cfg, sh.SH_DTYPE_F16, seed=121, std=0.08)
    assert check_steps(m, ref, sh.synth_tokens(16, 122, cfg.vocab)) < 1e-3
    m.close()


def test_eval_next_logits_repeatable_and_cache_reset(gpu):
    cfg = tiny_config()
    m, ref, _ = build(cfg, sh.SH_DTYPE_F16, seed=131, std=0.08)
    a, _ = m.eval_next_logits(5, 0)
    b, _ = m.eval_next_logits(7, 1)
    a2, _ = m.eval_next_logits(5, 0)
    np.testing.assert_array_equal(a, a2)
    m.reset_cache()
    b2, _ = m.eval_next_logits(7, 1)  # position 0 of the cache is zero now
    assert not np.array_equal(b, b2)
    with pytest.raises(sh.ShError):
        m.eval_next_logits(cfg.vocab, 0)
    with pytest.raises(sh.ShError):
        m.eval_next_logits(1, cfg.max_seq)
    m.close()


def test_greedy_decode_tiny_bookkeeping(gpu):
    cfg = tiny_config(max_seq=24)
    m, ref, w = build(cfg, sh.SH_DTYPE_F16, seed=141, std=0.08)
    p = sh.synth_tokens(5, 142, cfg.vocab)
    got, plen, eos = m.greedy_decode(p, 12)
    want, weos, _ = ref.greedy_decode(p, 12)
    assert plen == 5 and got.tolist() == want.tolist() and eos == weos
    # maxSeq stop, over-long prompt, empty prompt, invalid id (infer.go:152-163, :179)
    got, _, _ = m.greedy_decode(sh.synth_tokens(21, 143, cfg.vocab), 10)
    want, _, _ = ref.greedy_decode(sh.synth_tokens(21, 143, cfg.vocab), 10)
    assert len(got) == 24 and got.tolist() == want.tolist()
    long = sh.synth_tokens(30, 144, cfg.vocab)
    got, plen, _ = m.greedy_decode(long, 4)
    assert plen == 24 and got.tolist() == long[-24:].tolist()
    got, plen, _ = m.greedy_decode([], 3)
    want, _, _ = ref.greedy_decode([], 3)
    assert plen == 1 and got.tolist() == want.tolist()
    with pytest.raises(sh.ShError):
        m.greedy_decode([1, cfg.vocab + 3], 4)
    m.close()


def test_greedy_decode_stops_on_eos(gpu):
    cfg = tiny_config(max_seq=32, tied_embed=0)
    w = sh.synth_weights(cfg, seed=151, std=0.08)
    for lw in w.layers:
        for k in sh.LAYER_KEYS:
            lw[k] = np.zeros_like(lw[k])
    w.embed = np.full_like(w.embed, 0.01)
    w.cls = np.zeros_like(w.embed)
    w.cls[2] = 1.0  # every step's argmax is EOS=2
    m = sh.Model(cfg, sh.SH_DTYPE_F16)
    m.upload(w)
    got, _, eos = m.greedy_decode([5, 9, 11], 10)
    assert eos and got.tolist() == [5, 9, 11, 2]
    m.close()


def test_persistent_fallback_to_graph_path(gpu):
    """The persistent kernel's failure handling (engine.go:739-746 is the reference's contract:
    an accelerator failure switches to the other path and the call still answers). A launch
    whose grid was not all resident switches the model to the per-stage graph path and repeats
    the call there: the greedy stream and the next step's logits still match the oracle. A
    hand-over timeout with every workgroup running is an error and switches nothing. W8A8 has
    no per-stage path: a residency failure is an error."""
    cfg = tiny_config()
    prompt = sh.synth_tokens(6, 172, cfg.vocab)
    m, ref, _ = build(cfg, sh.SH_DTYPE_F16, seed=171, std=0.08)
    assert m.describe().startswith("persistent decode kernel")
    m.debug_fail_next_launch(2)
    got, plen, _ = m.greedy_decode(prompt, 12)
    want, _, want_logits = oracle_stream(ref, prompt, 12, cfg.max_seq)
    assert got.tolist() == want.tolist()
    assert not m.stats()["persistent"]
    assert "per-stage kernels" in m.describe() and "resident" in m.describe()
    check_stream(m, got, want_logits, tol=1e-3)
    m.close()
    # the same through sh_decode_step
    m, ref, _ = build(cfg, sh.SH_DTYPE_F16, seed=171, std=0.08)
    m.debug_fail_next_launch(2)
    got1, am = m.eval_next_logits(int(prompt[0]), 0)
    assert float(np.max(np.abs(got1 - ref.forward_one(int(prompt[0]), 0)))) < 1e-3
    assert not m.stats()["persistent"]
    m.close()
    # a timeout with every workgroup running: an error, the path kept, the next call fine
    m, ref, _ = build(cfg, sh.SH_DTYPE_F16, seed=171, std=0.08)
    m.debug_fail_next_launch(1)
    with pytest.raises(sh.ShError, match="every workgroup running"):
        m.greedy_decode(prompt, 12)
    assert m.describe().startswith("persistent decode kernel")
    got, _, _ = m.greedy_decode(prompt, 12)
    assert got.tolist() == want.tolist()
    m.close()
    # W8A8: no per-stage path
    m, ref, _ = build(cfg, sh.SH_DTYPE_W8A8, seed=171, std=0.08)
    m.debug_fail_next_launch(2)
    with pytest.raises(sh.ShError, match="not all resident"):
        m.greedy_decode(prompt, 12)
    m.close()


def test_calibration_kernels(gpu):
    """The copy and read-only stream kernels the bench lines quote as practical ceilings: both
    time a known byte count (64 MiB here) and refuse sizes that are not 16-byte multiples."""
    ms_c, copy_gbs = sh.copy_calibrate(64 << 20, reps=3)
    ms_r, read_gbs = sh.read_calibrate(64 << 20, reps=3)
    print(f"copy {copy_gbs:.0f} GB/s ({ms_c * 1e3:.1f} us), read {read_gbs:.0f} GB/s ({ms_r * 1e3:.1f} us)")
    assert ms_c > 0 and copy_gbs > 0 and ms_r > 0 and read_gbs > 0
    for f in (sh.copy_calibrate, sh.read_calibrate):
        with pytest.raises(sh.ShError, match="multiple of 16"):
            f(100, reps=1)


def test_quantize_bit_exact(gpu):
    rng = np.random.default_rng(161)
    w = (rng.standard_normal((300, 257)) * 0.02).astype(np.float32)
    w[7] = 0.0
    w[9, :5] = [1.0, -1.0, 0.5, -0.25, 3.0]
    s9 = np.float32(3.0) / np.float32(127.0)
    w[11, :4] = np.array([127.0, 0.5, -0.5, 2.5], np.float32) * (np.float32(1.0) / np.float32(127.0))
    q, s = sh.quantize_i8(w, per_row=True)
    qo, so = oracle.quantize_rows(w)
    np.testing.assert_array_equal(q, qo)
    np.testing.assert_array_equal(s.view(np.uint32), so.view(np.uint32))
    assert s[9] == s9 and s[7] == 1.0
    qt, st = sh.quantize_i8(w, per_row=False)
    qto, sto = oracle.quantize_tensor(w)
    np.testing.assert_array_equal(qt, qto)
    assert st[0] == sto
    dq = sh.dequantize_i8(q, s, per_row=True)
    np.testing.assert_array_equal(dq.view(np.uint32), oracle.dequantize_rows(qo, so).view(np.uint32))
    # empty and all-zero tensors: scale 1 (ane_bridge.m:383)
    qz, sz = sh.quantize_i8(np.zeros((4, 8), np.float32), per_row=False)
    assert sz[0] == 1.0 and not qz.any()


# ---- full-size configurations --------------------------------------------------------------

def check_stream(m, ids, want_logits, tol=LOGIT_TOL, exact=False):
    """Replays the token stream through sh_decode_step (one forward per position, cache
    reset first) and checks every forward's logits against the oracle's at that position:
    max-abs within tol (or bit-identical when exact) and the same first-max argmax."""
    m.reset_cache()
    worst = 0.0
    for pos in range(len(ids) - 1):
        got, am = m.eval_next_logits(int(ids[pos]), pos)
        want = want_logits[pos]
        if exact:
            assert np.array_equal(got, want), f"pos {pos}: max-abs {np.max(np.abs(got - want))}"
        err = float(np.max(np.abs(got - want)))
        worst = max(worst, err)
        assert err <= tol, f"pos {pos}: max-abs {err}"
        assert am == int(np.argmax(got)) == int(np.argmax(want)), f"pos {pos}"
    print(f"max-abs logits error over all {len(ids) - 1} forwards: {worst:.3e}")
    return worst


def test_stories110m_fp16_greedy_128(gpu):
    """Stories110M fp16 greedy decode: seed-0 N(0, 0.02) weights, 16-id prompt from seed 1,
    128 new tokens; token stream identical to the oracle's, and the logits of every one of
    the 143 forwards within max-abs 2e-2 of the oracle's."""
    cfg = sh.stories110m_config()
    m, ref, _ = build(cfg, sh.SH_DTYPE_F16, seed=0)
    prompt = sh.synth_tokens(16, 1, cfg.vocab)
    got, plen, eos = m.greedy_decode(prompt, 128)
    want, weos, want_logits = oracle_stream(ref, prompt, 128, cfg.max_seq)
    margins = top2_margins(want_logits[plen - 1:])
    print(f"generated {len(got) - plen} tokens; smallest top-2 margin {margins.min():.3e}")
    assert got.tolist() == want.tolist() and eos == weos
    assert len(got) == 16 + 128 or eos
    st = m.stats()
    print(f"persistent={st['persistent']} grid={st['grid']} {st['gpu_ms']:.3f} ms for {st['forwards']} forwards")
    assert st["persistent"]
    # a second decode reuses the model (epochs advance, cache is cleared)
    again, _, _ = m.greedy_decode(prompt, 128)
    assert again.tolist() == got.tolist()
    check_stream(m, got, want_logits)
    # the prompt fed through the token loop instead: the persistent launch runs the 15 prompt
    # forwards too (in this shape's layout the next token is exchanged after every forward)
    assert "from workgroup" in m.describe()
    m.set_prompt_prefill(False)
    got2, _, _ = m.greedy_decode(prompt, 128)
    assert got2.tolist() == want.tolist()
    assert m.stats()["forwards"] == 15 + 128   # no full-sequence forward ran
    m.close()


def test_qwen3_shaped_bf16_greedy(gpu):
    """Qwen3-0.6B-shaped bf16 decode (GQA 16/8, hd 128, QK-norm, theta 1e6, tied, bf16 KV):
    seed-3 weights, 32-id prompt from seed 3, 256 new tokens identical to the oracle's, and
    the logits of all 287 forwards within max-abs 2e-2."""
    cfg = sh.qwen3_06b_config()
    m, ref, _ = build(cfg, sh.SH_DTYPE_BF16, seed=3)
    prompt = sh.synth_tokens(32, 3, cfg.vocab)
    got, plen, eos = m.greedy_decode(prompt, 256)
    want, weos, want_logits = oracle_stream(ref, prompt, 256, cfg.max_seq)
    margins = top2_margins(want_logits[plen - 1:])
    print(f"generated {len(got) - plen} tokens; smallest top-2 margin {margins.min():.3e}")
    assert got.tolist() == want.tolist() and eos == weos
    st = m.stats()
    print(f"persistent={st['persistent']} grid={st['grid']} {st['gpu_ms']:.3f} ms for {st['forwards']} forwards")
    assert st["persistent"]
    check_stream(m, got, want_logits)
    # the prompt fed through the token loop: its 31 forwards run in the persistent launch, and
    # in this shape's layout (w13 on every workgroup) they skip the next-token exchange
    assert "from workgroup" not in m.describe()
    m.set_prompt_prefill(False)
    got2, _, _ = m.greedy_decode(prompt, 256)
    assert got2.tolist() == want.tolist()
    assert m.stats()["forwards"] == 31 + 256   # no full-sequence forward ran
    m.close()


SPECIAL = np.array([
    1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, -(1.0 + 2.0 ** -11),   # fp16 ties: to even
    1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8,                            # bf16 ties: to even
    1.5 * 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 0.75 * 2.0 ** -14,  # fp16 subnormals, ties
    65504.0, 65519.0, 65520.0, -70000.0, 0.0, -0.0, 1e-30, 3.0e38,   # range edges
], np.float64).astype(np.float32)


@pytest.mark.parametrize("dtype", [sh.SH_DTYPE_F16, sh.SH_DTYPE_BF16, sh.SH_DTYPE_W8A8])
def test_device_weight_rounding_is_bit_exact(gpu, dtype):
    """The device's conversion of uploaded fp32 weights, read back as stored: fp16 and bf16
    bits equal round-to-nearest-even (numpy's float16 conversion; the host helper
    sh_round_dtype for bf16), including ties, subnormals and overflow to infinity; W8A8 int8
    rows and row scales equal the oracle's bridge quantizer (ane_bridge.m:374-399) bit for
    bit. The reference's generic Go converter rounds halves up on magnitude
    (generator.go:151-219); the device follows its darwin path's hardware RNE
    (fp16_pack_darwin.go:11-35)."""
    cfg = tiny_config(tied_embed=0)
    w = sh.synth_weights(cfg, seed=171, std=0.05)
    lw = w.layers[1]
    lw["wq"][3, :SPECIAL.size] = SPECIAL
    lw["w3"][5, -SPECIAL.size:] = SPECIAL
    lw["w2"][7] = 0.0
    m = sh.Model(cfg, dtype)
    m.upload(w)
    for name in ("wq", "wk", "wv", "wo", "w1", "w2", "w3"):
        src = np.ascontiguousarray(lw[name], np.float32)
        got = m.read_weights(1, name)
        if dtype == sh.SH_DTYPE_F16:
            with np.errstate(over="ignore"):
                np.testing.assert_array_equal(got, src.astype(np.float16).view(np.uint16), err_msg=name)
        elif dtype == sh.SH_DTYPE_BF16:
            want = sh.round_dtype(src, sh.SH_DTYPE_BF16)
            assert np.array_equal(got.astype(np.uint32) << 16, want.view(np.uint32)), name
        else:
            q, sc = oracle.quantize_rows(src)
            np.testing.assert_array_equal(got, q, err_msg=name)
            np.testing.assert_array_equal(m.read_weights(1, name + ".scale").view(np.uint32), sc.view(np.uint32))
    # the embedding lookup table is 16-bit in every dtype (bf16 for BF16, else fp16)
    emb = m.read_weights(-1, "embed")
    e32 = np.ascontiguousarray(w.embed, np.float32)
    if dtype == sh.SH_DTYPE_BF16:
        want = sh.round_dtype(e32, sh.SH_DTYPE_BF16)
        assert np.array_equal(emb.astype(np.uint32) << 16, want.view(np.uint32))
    else:
        np.testing.assert_array_equal(emb, e32.astype(np.float16).view(np.uint16))
    with pytest.raises(sh.ShError):
        m.read_weights(cfg.n_layers, "wq")
    m.close()
