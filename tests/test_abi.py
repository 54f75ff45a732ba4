"""CPU checks of the C ABI: the library loads, exports every entry point declared in
include/stories_hip.h, and its host-only helpers behave (no device work here)."""
import os
import re

import numpy as np
import pytest
import torch

import stories_hip as sh

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "stories_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(sh_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    lib = sh.load()
    syms = header_symbols()
    assert len(syms) >= 18
    for name in syms:
        assert hasattr(lib, name), name
        assert name in sh.SIGNATURES, name


def test_stories_config_matches_reference_constants():
    c = sh.stories110m_config()
    # ane/stories/config.go:3-10; infer.go:102 (theta), :307 (eps)
    assert (c.dim, c.hidden, c.n_heads, c.n_layers, c.vocab, c.max_seq) == (768, 2048, 12, 12, 32000, 256)
    assert c.head_dim == 64 and c.n_kv_heads == 12 and c.rope_theta == 10000.0 and c.norm_eps == 1e-5
    assert c.residual_scale == 1.0 and c.tied_embed == 1 and c.qk_norm == 0
    q = sh.qwen3_06b_config()
    # training/training_dynamic/models/qwen3_06b.h:6-16
    assert (q.dim, q.hidden, q.n_heads, q.n_kv_heads, q.head_dim, q.n_layers, q.vocab) == \
        (1024, 3072, 16, 8, 128, 28, 151936)
    assert q.qk_norm == 1 and q.rope_theta == 1e6 and q.tied_embed == 1


def test_synthetic_normals_are_deterministic_and_normal():
    a = sh.synth_normal(200000, 0, 16, 0.02)
    b = sh.synth_normal(200000, 0, 16, 0.02)
    c = sh.synth_normal(200000, 0, 17, 0.02)
    d = sh.synth_normal(200000, 1, 16, 0.02)
    np.testing.assert_array_equal(a, b)
    assert not np.array_equal(a, c) and not np.array_equal(a, d)
    assert abs(a.mean()) < 2e-4 and abs(a.std() - 0.02) < 2e-4
    # Box-Muller: fourth moment of a normal is 3 sigma^4
    z = a.astype(np.float64) / 0.02
    assert abs(np.mean(z ** 4) - 3.0) < 0.1
    # prefix-stable: element i depends only on (seed, tensor id, i)
    np.testing.assert_array_equal(sh.synth_normal(1000, 0, 16, 0.02), a[:1000])


def test_synthetic_tokens_in_range():
    t = sh.synth_tokens(5000, 1, 32000)
    assert t.min() >= 0 and t.max() < 32000 and len(set(t.tolist())) > 4000
    np.testing.assert_array_equal(t, sh.synth_tokens(5000, 1, 32000))


def test_round_dtype_matches_library_casts():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(100000) * 10.0 ** rng.integers(-8, 4, 100000)).astype(np.float32)
    with np.errstate(over="ignore"):
        want16 = x.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(sh.round_dtype(x, sh.SH_DTYPE_F16).view(np.uint32), want16.view(np.uint32))
    wantbf = torch.tensor(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(sh.round_dtype(x, sh.SH_DTYPE_BF16).view(np.uint32), wantbf.view(np.uint32))


@pytest.mark.parametrize("field,value", [("head_dim", 48), ("n_kv_heads", 5), ("max_seq", 5000),
                                         ("dim", 100), ("hidden", 0), ("max_batch", 0)])
def test_invalid_configs_are_rejected_with_a_message(field, value):
    cfg = sh.stories110m_config()
    setattr(cfg, field, value)
    with pytest.raises(sh.ShError) as ei:
        sh.Model(cfg, sh.SH_DTYPE_F16)
    assert "invalid config" in str(ei.value)


def test_bad_dtype_rejected():
    with pytest.raises(sh.ShError):
        sh.Model(sh.stories110m_config(), 7)


def test_stateless_seams_reject_unsupported_shapes():
    lib = sh.load()
    e = np.zeros((100, 48), np.float32)
    x = np.zeros((48, 3), np.float32)
    out = np.zeros((100, 3), np.float32)
    fp = lambda a: a.ctypes.data_as(sh.C.POINTER(sh.C.c_float))
    assert lib.sh_matmul_vocab_seq(fp(e), fp(x), 100, 48, 3, fp(out)) == -1
    assert "dim % 32 == 0 and vocab % 64 == 0" in sh.last_error()
    assert lib.sh_matmul_vocab_seq(None, fp(x), 100, 48, 3, fp(out)) == -1
    assert "bad arguments" in sh.last_error()
    assert not lib.sh_conv_create(fp(e), 100, 48)
    assert "in_dim % 32 == 0 and out_dim % 64 == 0" in sh.last_error()
    assert lib.sh_conv_eval(None, fp(x), 3, fp(out)) == -1
    lib.sh_conv_destroy(None)


def test_trainer_refuses_unsupported_models_and_options():
    cfg = sh.make_config(dim=64, hidden=128, n_layers=1, n_heads=4, n_kv_heads=2, head_dim=16, vocab=96,
                         max_seq=32)
    with pytest.raises(sh.ShError, match="Stories-shaped"):
        sh.Trainer(cfg, seq=8)
    cfg.n_kv_heads = 4
    with pytest.raises(sh.ShError, match="seq must be <= 4096"):
        sh.Trainer(cfg, seq=8192, accum_steps=4)
    lib = sh.load()
    assert lib.sh_trainer_flush(None) == -1   # engine.go:399-401
    assert "engine is closed" in sh.last_error()
