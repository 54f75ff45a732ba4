"""CPU checks that pin the oracle's training step (ane/storiesane/train_full.go CPU path):
the reference's own known-answer tests for the cross-entropy and the embedding backward, the
gradients against torch float64 autograd of the same model (with the reference's two
deliberate shortcuts: q/k gradients are not rotated back through RoPE, and the classifier's
embedding gradient fills only the rows of target ids), Adam's first step in closed form,
gradient clipping's invariants, and the window RNG against the C library's drand48."""
import ctypes
import ctypes.util

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
import stories_hip as sh
from helpers import random_gains, tiny_config


def train_config(**kw):
    base = dict(dim=64, hidden=128, n_layers=2, n_heads=4, n_kv_heads=4, head_dim=16, vocab=96,
                max_seq=32, residual_scale=0.5)
    base.update(kw)
    return tiny_config(**base)


def setup(cfg, seed, seq=12, gains=False):
    w = sh.synth_weights(cfg, seed=seed, std=0.15)
    if gains:
        w = random_gains(w, seed + 1)
    toks = sh.synth_tokens(seq + 1, seed + 2, cfg.vocab)
    p = oracle.TrainParams.from_weights(w)
    return w, p, toks[:-1], toks[1:]


# ---- the reference's known-answer tests --------------------------------------------------

def test_cross_entropy_shape_and_zero_sum_columns():
    # ane/stories/cpu_test.go:8-33 TestCrossEntropyLossShape
    logits = np.array([[2, 0, -1], [0, 1, 0], [-1, 0, 2], [0, 0, 0]], np.float32)
    loss, d = oracle.cross_entropy_loss(logits, [0, 1, 2])
    assert loss > 0
    assert np.all(np.abs(d.sum(axis=0)) <= 1e-5)
    # the mean negative log-likelihood in float64
    z = logits.astype(np.float64)
    lp = z - np.log(np.exp(z - z.max(0)).sum(0)) - z.max(0)
    assert abs(loss - (-(lp[0, 0] + lp[1, 1] + lp[2, 2]) / 3)) <= 1e-6


def test_cross_entropy_out_of_range_target_skips_column():
    # ane/stories/cpu_test.go:76-104 TestCrossEntropyLossOutOfRangeTargetSkipsColumn
    logits = np.array([[2, 0], [0, 1], [-1, 0]], np.float32)
    loss, d = oracle.cross_entropy_loss(logits, [1, 99])
    assert loss > 0
    assert np.all(d[:, 1] == 0)
    assert abs(float(d[:, 0].sum())) <= 1e-5


def test_embed_backward_reference_case():
    # ane/stories/cpu_test.go:35-60 TestEmbedLookupBackward
    dim, seq, vocab = 3, 2, 5
    dx = np.array([1, 2, 3, 4, 5, 6], np.float32).reshape(dim, seq)
    de = np.zeros((vocab, dim), np.float32)
    oracle.embed_backward(de, dx, [1, 3])
    assert de[1].tolist() == [1, 3, 5] and de[3].tolist() == [2, 4, 6]
    assert not de[[0, 2, 4]].any()


def test_rms_backward_is_exact_for_unit_gains_and_off_by_the_gain_otherwise():
    # rmsnorm.go:32-47: dx = r*w*dy - (r^3/d) * x * w * (dy . (x*w)); the exact gradient of
    # y = x*r*w has no w factor on the second term. Autograd in float64 for both cases.
    rng = np.random.default_rng(5)
    d, s = 24, 7
    x = rng.standard_normal((d, s)).astype(np.float32)
    dy = rng.standard_normal((d, s)).astype(np.float32)
    r = (1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(0) + 1e-5)).astype(np.float32)
    for gain in (np.ones(d, np.float32), (0.5 + rng.random(d)).astype(np.float32)):
        dx, dw = oracle.rms_norm_backward_cf(dy, x, gain, r)
        xt = torch.tensor(x.T, dtype=torch.float64, requires_grad=True)
        wt = torch.tensor(gain, dtype=torch.float64, requires_grad=True)
        F.rms_norm(xt, (d,), wt, eps=1e-5).backward(torch.tensor(dy.T, dtype=torch.float64))
        exact = xt.grad.numpy().T
        xd, rd, gd = x.astype(np.float64), r.astype(np.float64), gain.astype(np.float64)[:, None]
        dot = (dy.astype(np.float64) * xd * gd).sum(0)
        quirk = (rd ** 3 / d) * xd * dot * (1 - gd)   # what the extra w factor changes
        np.testing.assert_allclose(dx, exact + quirk, atol=2e-5, rtol=0)
        np.testing.assert_allclose(dw, wt.grad.numpy(), atol=2e-5, rtol=0)
        if np.all(gain == 1):
            np.testing.assert_allclose(dx, exact, atol=2e-5, rtol=0)


# ---- gradients against float64 autograd (unit RMS gains, as RandomInit makes them) --------

class _RopeNoGrad(torch.autograd.Function):
    """RoPE forward; the gradient passes through unrotated (train_full.go:247-301 treats the
    post-RoPE q/k gradient as the projection's)."""

    @staticmethod
    def forward(ctx, t, rot):
        S, H, hd = t.shape
        c = torch.view_as_complex(t.reshape(S, H, hd // 2, 2).contiguous())
        return torch.view_as_real(c * rot[:, None, :]).reshape(S, H, hd)

    @staticmethod
    def backward(ctx, g):
        return g, None


def torch_grads_f64(cfg, w, inp, tgt):
    d = torch.float64
    S, H, hd, D = len(inp), cfg.n_heads, cfg.head_dim, cfg.dim
    a = cfg.residual_scale
    P = lambda x: torch.tensor(x, dtype=d, requires_grad=True)
    layers = [{k: P(l[k]) for k in oracle.TRAIN_KEYS} for l in w.layers]
    E, G = P(w.embed), P(w.rms_final)
    pos = torch.arange(S, dtype=d)
    inv_freq = torch.tensor([cfg.rope_theta ** (-(2.0 * i) / hd) for i in range(hd // 2)], dtype=d)
    rot = torch.polar(torch.ones(S, hd // 2, dtype=d), pos[:, None] * inv_freq[None, :])
    x = E[torch.tensor(np.asarray(inp, np.int64))]
    for L in layers:
        xn = F.rms_norm(x, (D,), L["rms_att"], eps=cfg.norm_eps)
        q = _RopeNoGrad.apply((xn @ L["wq"].T).reshape(S, H, hd), rot)
        k = _RopeNoGrad.apply((xn @ L["wk"].T).reshape(S, H, hd), rot)
        v = (xn @ L["wv"].T).reshape(S, H, hd)
        att = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1),
                                             is_causal=True).transpose(0, 1).reshape(S, D)
        x2 = x + a * (att @ L["wo"].T)
        x2n = F.rms_norm(x2, (D,), L["rms_ffn"], eps=cfg.norm_eps)
        x = x2 + a * ((F.silu(x2n @ L["w1"].T) * (x2n @ L["w3"].T)) @ L["w2"].T)
    xnf = F.rms_norm(x, (D,), G, eps=cfg.norm_eps)
    rows = torch.zeros(cfg.vocab, 1, dtype=d)
    rows[torch.tensor(sorted(set(int(t) for t in tgt if t < cfg.vocab)))] = 1
    Ecls = E * rows + E.detach() * (1 - rows)   # classifier gradient on target rows only
    logits = xnf @ Ecls.T
    loss = F.cross_entropy(logits, torch.tensor(np.asarray(tgt, np.int64)))
    loss.backward()
    grads = {}
    for i, L in enumerate(layers):
        for k in oracle.TRAIN_KEYS:
            grads[f"layers.{i}.{k}"] = L[k].grad.numpy()
    grads["embed"], grads["rms_final"] = E.grad.numpy(), G.grad.numpy()
    return loss.item(), grads


@pytest.mark.parametrize("loss_scale", [256.0, 1.0])
def test_train_gradients_match_float64_autograd(loss_scale):
    cfg = train_config()
    w, p, inp, tgt = setup(cfg, 201)
    m, v, g = (oracle.TrainParams.zeros_like(p) for _ in range(3))
    loss = oracle.train_step(oracle.config_from(cfg), p, m, v, g, oracle.hparams(loss_scale=loss_scale), 1,
                             inp, tgt, apply=False, threads=2)
    ref_loss, ref = torch_grads_f64(cfg, w, inp, tgt)
    assert abs(loss - ref_loss) <= 2e-6 * max(1.0, ref_loss)
    for name, got in g.tensors():
        want = ref[name]
        err = float(np.max(np.abs(got - want))) / max(float(np.max(np.abs(want))), 1e-30)
        assert err <= 2e-4, (name, err)


def test_adam_first_step_closed_form():
    # step 1 from zero moments: bias correction makes m_hat = g and v_hat = g^2, so each
    # weight moves by lr * (g / (|g| + eps) + wd * w), without the decay for the RMS gains
    cfg = train_config()
    w, p, inp, tgt = setup(cfg, 211)
    before = {n: a.copy() for n, a in p.tensors()}
    m, v, g = (oracle.TrainParams.zeros_like(p) for _ in range(3))
    hp = oracle.hparams(lr=1e-3, weight_decay=0.1)
    oracle.train_step(oracle.config_from(cfg), p, m, v, g, hp, 1, inp, tgt, apply=True, threads=2)
    grads = dict(g.tensors())
    for name, after in p.tensors():
        w0, gg = before[name].astype(np.float64), grads[name].astype(np.float64)
        wd = 0.0 if name.endswith(("rms_att", "rms_ffn")) or name == "rms_final" else 0.1
        want = w0 - 1e-3 * (gg / (np.abs(gg) + 1e-8) + wd * w0)
        assert float(np.max(np.abs(after - want))) <= 1e-6, name


def test_gradient_clipping_scales_to_the_bound():
    cfg = train_config()
    _, p, inp, tgt = setup(cfg, 221)
    ocfg = oracle.config_from(cfg)
    g0 = oracle.TrainParams.zeros_like(p)
    z = lambda: oracle.TrainParams.zeros_like(p)
    oracle.train_step(ocfg, p, z(), z(), g0, oracle.hparams(), 1, inp, tgt, apply=False)
    g1 = oracle.TrainParams.zeros_like(p)
    oracle.train_step(ocfg, p, z(), z(), g1, oracle.hparams(grad_clip=1e-3), 1, inp, tgt, apply=False)
    a = np.concatenate([x.ravel() for _, x in g0.tensors()]).astype(np.float64)
    b = np.concatenate([x.ravel() for _, x in g1.tensors()]).astype(np.float64)
    assert np.linalg.norm(a) > 1e-3
    assert abs(np.linalg.norm(b) - 1e-3) <= 1e-8
    np.testing.assert_allclose(b, a * (1e-3 / np.linalg.norm(a)), rtol=1e-5, atol=1e-12)


def test_loss_falls_over_steps_on_one_window():
    cfg = train_config()
    _, p, inp, tgt = setup(cfg, 231)
    m, v, g = (oracle.TrainParams.zeros_like(p) for _ in range(3))
    ocfg = oracle.config_from(cfg)
    losses = [oracle.train_step(ocfg, p, m, v, g, oracle.hparams(lr=3e-3), t, inp, tgt, threads=2)
              for t in range(1, 7)]
    assert losses[-1] < losses[0] - 0.05 and all(np.isfinite(losses))


def test_window_rng_is_drand48():
    libc = ctypes.CDLL(ctypes.util.find_library("c"))
    libc.drand48.restype = ctypes.c_double
    L = oracle.load()
    for seed in (42, 7, 123456789):
        libc.srand48(ctypes.c_long(seed))
        st = ctypes.c_uint64(L.or_drand48_seed(seed))
        for _ in range(5):
            assert L.or_drand48_next(ctypes.byref(st)) == libc.drand48()
    # Step's window (engine.go:307-316): floor(u * limit), limit = n - seq - 1
    st = ctypes.c_uint64(L.or_drand48_seed(42))
    st2 = ctypes.c_uint64(L.or_drand48_seed(42))
    for _ in range(4):
        u = L.or_drand48_next(ctypes.byref(st2))
        assert L.or_train_window(ctypes.byref(st), 1000, 256) == int(u * (1000 - 256 - 1))


# ---- gradient accumulation (backwardAndAccumulate + flushPending) -------------------------

def test_accumulate_one_window_then_flush_is_the_plain_step():
    # with one pending window the flush scale float32(1)/256 is the plain step's 1/256, and
    # adding onto zero sums changes nothing: the result is bit-identical
    cfg = train_config()
    ocfg = oracle.config_from(cfg)
    _, p1, inp, tgt = setup(cfg, 241, gains=True)
    _, p2, _, _ = setup(cfg, 241, gains=True)
    hp = oracle.hparams(lr=1e-3, weight_decay=0.1, grad_clip=5e-2)
    m1, v1, g1 = (oracle.TrainParams.zeros_like(p1) for _ in range(3))
    m2, v2, acc = (oracle.TrainParams.zeros_like(p2) for _ in range(3))
    l1 = oracle.train_step(ocfg, p1, m1, v1, g1, hp, 1, inp, tgt, threads=2)
    l2 = oracle.train_accumulate(ocfg, p2, acc, hp, inp, tgt, threads=2)
    oracle.train_flush(ocfg, p2, m2, v2, acc, hp, 1, 1)
    assert l1 == l2
    for a, b in ((p1, p2), (m1, m2), (v1, v2), (g1, acc)):
        for (name, x), (_, y) in zip(a.tensors(), b.tensors()):
            assert np.array_equal(x, y), name


def test_accumulated_sums_are_the_sum_of_window_gradients():
    # d(L_a + L_b) = dL_a + dL_b: the accumulator after two windows against the plain step's
    # gradients of each (times the loss scale, a power of two). Products and the embedding and
    # final-gain rows add once per window, exactly; the layer gains' sums continue over the
    # second window's rows (rmsNormBackward into the accumulator), a rounding-level difference.
    cfg = train_config()
    ocfg = oracle.config_from(cfg)
    _, p, inp, tgt = setup(cfg, 251, gains=True)
    toks_b = sh.synth_tokens(13, 252, cfg.vocab)
    hp = oracle.hparams()
    z = lambda: oracle.TrainParams.zeros_like(p)
    ga, gb, acc = z(), z(), z()
    oracle.train_step(ocfg, p, z(), z(), ga, hp, 1, inp, tgt, apply=False)
    oracle.train_step(ocfg, p, z(), z(), gb, hp, 1, toks_b[:-1], toks_b[1:], apply=False)
    oracle.train_accumulate(ocfg, p, acc, hp, inp, tgt)
    oracle.train_accumulate(ocfg, p, acc, hp, toks_b[:-1], toks_b[1:])
    for (name, a), (_, b), (_, s) in zip(ga.tensors(), gb.tensors(), acc.tensors()):
        want = a * np.float32(256) + b * np.float32(256)
        if name.endswith(("rms_att", "rms_ffn")):
            np.testing.assert_allclose(s, want, rtol=1e-5, atol=1e-7 * float(np.max(np.abs(want))), err_msg=name)
        else:
            assert np.array_equal(s, want), name


def test_flush_of_a_repeated_window_is_one_plain_step():
    # the mean of two identical windows is that window's gradient: scale 1/(2*256) is exact,
    # so products, embedding and final gain match the plain step bit for bit
    cfg = train_config()
    ocfg = oracle.config_from(cfg)
    _, p1, inp, tgt = setup(cfg, 261)
    _, p2, _, _ = setup(cfg, 261)
    hp = oracle.hparams(lr=1e-3)
    m1, v1, g1 = (oracle.TrainParams.zeros_like(p1) for _ in range(3))
    m2, v2, acc = (oracle.TrainParams.zeros_like(p2) for _ in range(3))
    oracle.train_step(ocfg, p1, m1, v1, g1, hp, 1, inp, tgt)
    oracle.train_accumulate(ocfg, p2, acc, hp, inp, tgt)
    oracle.train_accumulate(ocfg, p2, acc, hp, inp, tgt)
    oracle.train_flush(ocfg, p2, m2, v2, acc, hp, 1, 2)
    for (name, a), (_, b) in zip(p1.tensors(), p2.tensors()):
        if name.endswith(("rms_att", "rms_ffn")):
            assert float(np.max(np.abs(a - b))) <= 1e-6, name
        else:
            assert np.array_equal(a, b), name


def test_flush_pending_reference_case():
    # ane/storiesane/engine_test.go:107-152 TestFlushPendingAppliesUpdate: two pending windows,
    # lr 1e-3, loss scale, betas and eps zero, no layers. Adam's step 1 with beta 0 is
    # w - lr * g/|g|, and the applied gradients are the sums halved. (The reference's embedding
    # has 3 values against a 2-value gain; here dim 2, vocab 2.)
    c = oracle.OrConfig()
    c.dim, c.vocab, c.n_layers = 2, 2, 0
    p = oracle.TrainParams([], np.array([[1, 2], [3, 4]], np.float32), np.array([1, 1], np.float32))
    acc = oracle.TrainParams([], np.array([[3, 6], [9, 12]], np.float32), np.array([2, 4], np.float32))
    m, v = oracle.TrainParams.zeros_like(p), oracle.TrainParams.zeros_like(p)
    hp = oracle.hparams(lr=1e-3, beta1=0.0, beta2=0.0, eps=0.0, loss_scale=0.0)
    oracle.train_flush(c, p, m, v, acc, hp, 1, 2)
    lr = np.float32(1e-3)
    assert np.array_equal(p.rms_final, np.float32(1) - lr * np.ones(2, np.float32))
    assert np.array_equal(p.embed, np.array([[1, 2], [3, 4]], np.float32) - lr)
    assert acc.rms_final.tolist() == [1, 2] and acc.embed.tolist() == [[1.5, 3], [4.5, 6]]
    # nothing pending: no update
    oracle.train_flush(c, p, m, v, acc, hp, 2, 0)
    assert np.array_equal(p.rms_final, np.float32(1) - lr * np.ones(2, np.float32))


def test_rms_grad_weights_reference_fixture():
    # ane/storiesane/engine_test.go:376-400 TestRMSNormGradWeightsMatchesCPUBackward: dim 3,
    # seq 2, its dy / x / w; dw[i] = sum_t dy*x*rrms_t with rrms_t = 1/sqrt(mean_i x^2 + 1e-5)
    dy = np.array([[0.1, 0.2], [0.3, 0.4], [0.5, 0.6]], np.float32)
    x = np.array([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], np.float32)
    w = np.array([1.1, 0.9, 1.2], np.float32)
    r = (1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(0) + 1e-5)).astype(np.float32)
    _, dw = oracle.rms_norm_backward_cf(dy, x, w, r)
    want = (dy.astype(np.float64) * x.astype(np.float64) * r.astype(np.float64)).sum(1)
    np.testing.assert_allclose(dw, want, atol=1e-5, rtol=0)


def test_cross_entropy_reference_fixture():
    # ane/storiesane/engine_test.go:402-448 TestCrossEntropyLossFromProbsMatchesCPU: vocab 4,
    # seq 3, targets (3, 2, 9) with 9 out of range; loss and gradient against float64
    logits = np.array([[0.4, -0.2, 1.3], [0.1, 0.7, -0.1], [-0.3, 0.5, 0.2], [1.0, -0.4, 0.0]], np.float32)
    tg = [3, 2, 9]
    loss, d = oracle.cross_entropy_loss(logits, tg)
    z = logits.astype(np.float64)
    p = np.exp(z - z.max(0)) / np.exp(z - z.max(0)).sum(0)
    want_loss = -(np.log(p[3, 0]) + np.log(p[2, 1])) / 2
    g = p.copy()
    g[3, 0] -= 1
    g[2, 1] -= 1
    g[:, :2] /= 2
    g[:, 2] = 0
    assert abs(loss - want_loss) <= 1e-5
    np.testing.assert_allclose(d, g, atol=1e-5, rtol=0)
