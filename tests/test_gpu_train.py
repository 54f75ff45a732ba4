"""GPU parity of the training step (storiesane Engine.Step: train_full.go forwardTraining,
runFinalHead and backwardAndApply, or backwardAndAccumulate with flushPending, CPU-path
numerics) against the oracle's restatement, through the C ABI.

Bar: fp32 on both sides, differing only in summation order. The loss within 2e-5 relative;
every gradient Adam applies within 1e-3 of its tensor's largest magnitude (summation order
over the sequence and the fused W1|W3 / Wq|Wk|Wv products); the device's Adam step equal to
its closed form (step 1: w - lr*(g/(|g|+eps) + wd*w)) on the device's own gradients within
1e-6; and the weights against the oracle's: Adam's first step is g/(|g|+eps), which turns
rounding-level gradient differences into up to 2*lr where |g| is near eps, so per Adam step
at most 1e-4 of the elements may differ by more than 1e-6, and none by more than 2*lr. Three
Step() calls over drand48 windows of a token stream give the same windows and losses."""
import os

import numpy as np
import pytest

import oracle
import stories_hip as sh
from helpers import tiny_config

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))


def train_config(**kw):
    base = dict(dim=64, hidden=128, n_layers=2, n_heads=4, n_kv_heads=4, head_dim=16, vocab=96,
                max_seq=32, residual_scale=0.5)
    base.update(kw)
    return tiny_config(**base)


def wide_train_config():
    """A shape whose products have K >= 512 (W2's K = hidden = 512, the W1|W3 input gradient
    K = 1024, the classifier input gradient K = vocab = 1024), so the split-K products hand
    their partials to the row kernels (RMSNorm forward and backward, RoPE, SiLU backward),
    and head_dim 32 takes the MFMA attention kernels."""
    return train_config(dim=128, hidden=512, n_heads=4, n_kv_heads=4, head_dim=32, vocab=1024,
                        max_seq=64)


CONFIGS = {"tiny": train_config, "wide": wide_train_config}


def make(cfg, wseed, seq, std=0.15, **opts):
    w = sh.synth_weights(cfg, seed=wseed, std=std)
    tr = sh.Trainer(cfg, seq=seq, **opts)
    tr.upload(w)
    return w, tr


def compare_weights(tr, ref: oracle.TrainParams, steps, lr):
    """Weights against the oracle's after `steps` Adam steps: at most 1e-4 of the elements per
    step beyond 1e-6 (each step amplifies its own near-eps gradients), none beyond 2*lr per step."""
    n = far = 0
    for name, want in ref.tensors():
        got = tr.read(sh.SH_TRAIN_PARAMS, name, want.shape)
        d = np.abs(got - want)
        assert float(d.max()) <= 2 * lr * steps, (name, float(d.max()))
        n += d.size
        far += int((d > 1e-6).sum())
    print(f"weights: {far} of {n} elements differ by more than 1e-6")
    assert far <= 1e-4 * n * steps


def check_adam_closed_form(tr, before: dict, lr, wd, eps=1e-8):
    """Step 1 from zero moments on the device's own gradients: w - lr*(g/(|g|+eps) + wd*w)."""
    for name, w0 in before.items():
        g = tr.read(sh.SH_TRAIN_GRADS, name, w0.shape).astype(np.float64)
        got = tr.read(sh.SH_TRAIN_PARAMS, name, w0.shape)
        d = 0.0 if name.endswith(("rms_att", "rms_ffn")) or name == "rms_final" else wd
        want = w0.astype(np.float64) - lr * (g / (np.abs(g) + eps) + d * w0.astype(np.float64))
        assert float(np.max(np.abs(got - want))) <= 1e-6, name


def compare_tensors(tr, ref: oracle.TrainParams, which, atol=None, rel=None):
    worst = 0.0
    for name, want in ref.tensors():
        got = tr.read(which, name, want.shape)
        scale = max(float(np.max(np.abs(want))), 1e-30)
        err = float(np.max(np.abs(got - want)))
        if rel is not None:
            assert err <= rel * scale, (name, err, scale)
        if atol is not None:
            assert err <= atol, (name, err)
        worst = max(worst, err / scale)
    return worst


@pytest.mark.parametrize("kind,seq,clip,wd", [("tiny", 12, 0.0, 0.0), ("tiny", 40, 1e-2, 0.1),
                                               ("wide", 48, 1e-2, 0.1)])
def test_train_step_matches_oracle(gpu, kind, seq, clip, wd):
    cfg = CONFIGS[kind]()
    w, tr = make(cfg, 301, seq, lr=1e-3, grad_clip=clip, weight_decay=wd)
    toks = sh.synth_tokens(seq + 1, 302, cfg.vocab)
    inp, tgt = toks[:-1], toks[1:]
    p = oracle.TrainParams.from_weights(w)
    before = dict((n, a.copy()) for n, a in p.tensors())
    loss = tr.step_window(inp, tgt)
    m, v, g = (oracle.TrainParams.zeros_like(p) for _ in range(3))
    want = oracle.train_step(oracle.config_from(cfg), p, m, v, g,
                             oracle.hparams(lr=1e-3, grad_clip=clip, weight_decay=wd), 1, inp, tgt, threads=THREADS)
    print(f"seq {seq}: loss {loss:.6f} vs {want:.6f}")
    assert abs(loss - want) <= 2e-5 * abs(want)
    gerr = compare_tensors(tr, g, sh.SH_TRAIN_GRADS, rel=1e-3)
    print(f"worst gradient error {gerr:.2e} (relative to the tensor's max)")
    compare_tensors(tr, m, sh.SH_TRAIN_ADAM_M, rel=1e-3)
    check_adam_closed_form(tr, before, 1e-3, wd)
    compare_weights(tr, p, 1, 1e-3)
    assert tr.state()["adam_t"] == 1
    tr.close()


def test_engine_steps_follow_the_drand48_windows(gpu):
    cfg = train_config()
    seq = 16
    w, tr = make(cfg, 311, seq, lr=1e-3, seed=7)
    stream = sh.synth_tokens(200, 312, cfg.vocab)
    tr.set_tokens(stream)
    p = oracle.TrainParams.from_weights(w)
    m, v, g = (oracle.TrainParams.zeros_like(p) for _ in range(3))
    L = oracle.load()
    st = oracle.C.c_uint64(L.or_drand48_seed(7))
    ocfg = oracle.config_from(cfg)
    for t in range(1, 4):
        pos = L.or_train_window(oracle.C.byref(st), stream.size, seq)
        want = oracle.train_step(ocfg, p, m, v, g, oracle.hparams(lr=1e-3), t, stream[pos:pos + seq],
                                 stream[pos + 1:pos + 1 + seq], threads=THREADS)
        got = tr.step()
        assert abs(got - want) <= 2e-5 * abs(want), (t, got, want)
        assert tr.state()["token_pos"] == pos + seq
    compare_weights(tr, p, 3, 1e-3)
    assert tr.state()["cum_steps"] == 3 and tr.state()["adam_t"] == 3
    tr.close()


@pytest.mark.parametrize("seq", [64, 256])
def test_stories110m_train_step_matches_oracle(gpu, seq):
    """Stories110M shape (dim 768, 12 layers, vocab 32000), the engine's residual scale
    1/sqrt(24), a 64-token window and the benchmark's 256-token window: the loss, every
    gradient Adam applies, and a sample of the updated weights."""
    cfg = sh.stories110m_config()
    cfg.residual_scale = 1.0 / np.sqrt(24.0)
    w, tr = make(cfg, 321, seq, std=0.02, lr=3e-4)
    toks = sh.synth_tokens(seq + 1, 322, cfg.vocab)
    p = oracle.TrainParams.from_weights(w)
    sample = ("layers.0.wq", "layers.5.w2", "layers.11.wo", "layers.11.rms_ffn", "rms_final", "embed")
    before = {n: a.copy() for n, a in p.tensors() if n in sample}
    loss = tr.step_window(toks[:-1], toks[1:])
    m, v, g = (oracle.TrainParams.zeros_like(p) for _ in range(3))
    want = oracle.train_step(oracle.config_from(cfg), p, m, v, g, oracle.hparams(lr=3e-4), 1, toks[:-1],
                             toks[1:], threads=THREADS)
    print(f"Stories110M S={seq}: loss {loss:.6f} vs {want:.6f}, step {tr.state()['last_step_ms']:.2f} ms")
    assert abs(loss - want) <= 2e-5 * abs(want)
    gerr = compare_tensors(tr, g, sh.SH_TRAIN_GRADS, rel=1e-3)
    print(f"worst gradient error {gerr:.2e} (relative to the tensor's max)")
    # the update is Adam's first step on the device's own gradients (exact), and against the
    # oracle's weights it differs only where |g| is near eps, where g/(|g|+eps) magnifies
    # rounding-level gradient differences (more such elements in a longer window)
    check_adam_closed_form(tr, before, 3e-4, 0.0)
    params = dict(p.tensors())
    for name in sample:
        got = tr.read(sh.SH_TRAIN_PARAMS, name, params[name].shape)
        d = np.abs(got - params[name])
        assert float(d.max()) <= 2 * 3e-4 and int((d > 1e-6).sum()) <= 5e-4 * d.size + 1, name
    tr.close()


@pytest.mark.parametrize("kind", ["tiny", "wide"])
def test_gradient_accumulation_matches_oracle(gpu, kind):
    """AccumSteps 2 (backwardAndAccumulate, flushPending) over five windows: the pending sums
    after one window, the applied mean gradients and the weights after each flush, then a
    window flushed early by Flush(), and a Flush() with nothing pending."""
    cfg = CONFIGS[kind]()
    seq, lr, clip = 12, 1e-3, 1e-2
    w, tr = make(cfg, 341, seq, lr=lr, grad_clip=clip, accum_steps=2)
    p = oracle.TrainParams.from_weights(w)
    before = dict((n, a.copy()) for n, a in p.tensors())
    m, v, acc = (oracle.TrainParams.zeros_like(p) for _ in range(3))
    ocfg, hp = oracle.config_from(cfg), oracle.hparams(lr=lr, grad_clip=clip)
    stream = sh.synth_tokens(5 * (seq + 1), 342, cfg.vocab)
    wins = [(stream[i * (seq + 1):(i + 1) * (seq + 1) - 1], stream[i * (seq + 1) + 1:(i + 1) * (seq + 1)])
            for i in range(5)]
    t = 0
    for k, (inp, tgt) in enumerate(wins[:4]):
        got = tr.step_window(inp, tgt)
        want = oracle.train_accumulate(ocfg, p, acc, hp, inp, tgt, threads=THREADS)
        assert abs(got - want) <= 2e-5 * abs(want), (k, got, want)
        st = tr.state()
        if k % 2 == 0:
            assert st["pending_steps"] == 1 and st["adam_t"] == t
            compare_tensors(tr, acc, sh.SH_TRAIN_GRADS, rel=1e-3)   # the pending sums
            if k == 0:
                for name, w0 in before.items():   # no update yet
                    assert np.array_equal(tr.read(sh.SH_TRAIN_PARAMS, name, w0.shape), w0), name
        else:
            t += 1
            oracle.train_flush(ocfg, p, m, v, acc, hp, t, 2)
            assert st["pending_steps"] == 0 and st["adam_t"] == t and st["cum_batches"] == t
            compare_tensors(tr, acc, sh.SH_TRAIN_GRADS, rel=1e-3)   # the applied gradients
            if t == 1:
                check_adam_closed_form(tr, before, lr, 0.0)
            compare_weights(tr, p, t, lr)
            acc.clear()
    inp, tgt = wins[4]
    tr.step_window(inp, tgt)
    oracle.train_accumulate(ocfg, p, acc, hp, inp, tgt, threads=THREADS)
    assert tr.state()["pending_steps"] == 1
    tr.flush()
    oracle.train_flush(ocfg, p, m, v, acc, hp, 3, 1)
    st = tr.state()
    assert st["pending_steps"] == 0 and st["adam_t"] == 3 and st["cum_batches"] == 3 and st["cum_steps"] == 5
    compare_weights(tr, p, 3, lr)
    snap = tr.read(sh.SH_TRAIN_PARAMS, "layers.0.wq", (cfg.dim, cfg.dim))
    tr.flush()   # nothing pending: no change
    assert tr.state()["adam_t"] == 3
    assert np.array_equal(tr.read(sh.SH_TRAIN_PARAMS, "layers.0.wq", (cfg.dim, cfg.dim)), snap)
    tr.close()


def test_twenty_step_loss_delta_gate(gpu):
    """The reference's training parity gate (scripts/pure_go_parity_gate.sh:13-14: 20 steps,
    max loss delta 0.01 between implementations): 20 Step() calls over drand48 windows, device
    against oracle, every loss within 0.01 (and the losses fall)."""
    cfg = train_config()
    seq = 16
    w, tr = make(cfg, 351, seq, lr=3e-3, seed=11)
    stream = sh.synth_tokens(400, 352, cfg.vocab)
    tr.set_tokens(stream)
    p = oracle.TrainParams.from_weights(w)
    m, v, g = (oracle.TrainParams.zeros_like(p) for _ in range(3))
    L = oracle.load()
    st = oracle.C.c_uint64(L.or_drand48_seed(11))
    ocfg, hp = oracle.config_from(cfg), oracle.hparams(lr=3e-3)
    worst, got_all = 0.0, []
    for t in range(1, 21):
        pos = L.or_train_window(oracle.C.byref(st), stream.size, seq)
        want = oracle.train_step(ocfg, p, m, v, g, hp, t, stream[pos:pos + seq], stream[pos + 1:pos + 1 + seq],
                                 threads=THREADS)
        got = tr.step()
        got_all.append(got)
        worst = max(worst, abs(got - want))
    print(f"20 steps: max loss delta {worst:.2e}, loss {got_all[0]:.4f} -> {got_all[-1]:.4f}")
    assert worst <= 0.01
    assert np.mean(got_all[-5:]) < np.mean(got_all[:5])
    tr.close()


def test_train_errors(gpu):
    cfg = train_config()
    _, tr = make(cfg, 331, 16)
    tr.set_tokens(np.arange(10, dtype=np.uint16))
    with pytest.raises(sh.ShError, match="not enough tokens"):
        tr.step()
    with pytest.raises(sh.ShError, match="unknown tensor"):
        tr.read(sh.SH_TRAIN_PARAMS, "layers.9.wq", (64, 64))
    tr.close()
