"""GPU parity of the full-window greedy decode ((*Engine).Decode with Temperature 0,
ane/storiesane/decode.go:18-94) against the oracle: each step is the oracle's channel-first
forward (engine.go:804-842) of the BOS-padded window (fillDecodeWindow, decode.go:83-94),
then the first maximum of the last column. Bar: identical token streams."""
import math
import os

import numpy as np
import pytest

import oracle
import stories_hip as sh
from helpers import deepnet_alpha, tiny_config

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))


def oracle_window_decode(ocfg, ow, prompt, seq, max_new):
    toks = list(prompt) if len(prompt) else [1]
    toks = toks[-seq:]
    plen = len(toks)
    margins = []
    for _ in range(max_new):
        window = oracle.fill_decode_window(seq, np.asarray(toks, np.int32))
        logits = oracle.eval_logits_cf(ocfg, ow, window, threads=THREADS)[:, seq - 1]
        top2 = np.sort(logits)[-2:]
        margins.append(float(top2[1] - top2[0]))
        nxt = int(np.argmax(logits))
        toks.append(nxt)
        if nxt == 2:
            break
    return np.array(toks, np.int32), plen, min(margins)


def build(cfg, seed, std):
    w = sh.synth_weights(cfg, seed=seed, std=std)
    m = sh.Model(cfg, sh.SH_DTYPE_F16)
    m.upload(w)
    return m, oracle.config_from(cfg), w.rounded(sh.SH_DTYPE_F16)


def test_window_decode_tiny(gpu):
    cfg = tiny_config(n_layers=2, residual_scale=deepnet_alpha(2))
    m, ocfg, ow = build(cfg, 701, 0.08)
    for prompt, seq, steps in ((sh.synth_tokens(5, 702, cfg.vocab), 16, 20),
                               (sh.synth_tokens(40, 703, cfg.vocab), 16, 12),   # window slides
                               (np.zeros(0, np.int32), 8, 10)):                # empty -> [BOS]
        got, plen, eos = m.window_greedy_decode(prompt, seq, steps)
        want, wplen, margin = oracle_window_decode(ocfg, ow, prompt, seq, steps)
        print(f"seq {seq}: {len(got) - plen} tokens, smallest margin {margin:.3e}, "
              f"{m.stats()['gpu_ms']:.3f} ms")
        assert plen == wplen and got.tolist() == want.tolist()
        assert eos == (want[-1] == 2 and len(want) - wplen <= steps)
    with pytest.raises(sh.ShError):
        m.window_greedy_decode([1, cfg.vocab], 16, 4)
    with pytest.raises(sh.ShError):
        m.window_greedy_decode([1, 2], cfg.max_seq + 1, 4)
    m.close()


def test_window_decode_stops_on_eos(gpu):
    cfg = tiny_config(tied_embed=0)
    w = sh.synth_weights(cfg, seed=711, std=0.08)
    for lw in w.layers:
        for k in sh.LAYER_KEYS:
            lw[k] = np.zeros_like(lw[k])
    w.embed = np.full_like(w.embed, 0.01)
    w.cls = np.zeros_like(w.embed)
    w.cls[2] = 1.0
    m = sh.Model(cfg, sh.SH_DTYPE_F16)
    m.upload(w)
    got, plen, eos = m.window_greedy_decode([5, 9], 8, 10)
    assert eos and got.tolist() == [5, 9, 2]
    m.close()


def test_window_decode_stories110m(gpu):
    """Stories110M fp16 with the engine's residual scale 1/sqrt(24): a 256-token window over a
    16-id prompt from seed 1, 6 steps."""
    cfg = sh.stories110m_config()
    cfg.residual_scale = 1.0 / math.sqrt(24.0)
    m, ocfg, ow = build(cfg, 0, 0.02)
    prompt = sh.synth_tokens(16, 1, cfg.vocab)
    got, plen, _ = m.window_greedy_decode(prompt, 256, 6)
    want, _, margin = oracle_window_decode(ocfg, ow, prompt, 256, 6)
    print(f"smallest margin {margin:.3e}; {m.stats()['gpu_ms'] / 6:.3f} ms per step")
    assert got.tolist() == want.tolist()
    m.close()
