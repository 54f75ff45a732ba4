"""Helpers shared by the test modules: small model shapes, synthetic weights and an
independent float64 forward written with torch library routines (rms_norm, silu,
scaled_dot_product_attention, complex-number RoPE) used to pin the oracle."""
import math

import numpy as np
import torch
import torch.nn.functional as F

import stories_hip as sh


def tiny_config(**kw):
    """A small Llama shape that every kernel tiling supports."""
    base = dict(dim=128, hidden=256, n_layers=2, n_heads=4, n_kv_heads=4, head_dim=32,
                vocab=512, max_seq=64, rope_theta=10000.0, norm_eps=1e-5, qk_norm_eps=1e-6,
                residual_scale=1.0, qk_norm=0, tied_embed=1, kv_dtype=sh.SH_KV_F32, max_batch=1)
    base.update(kw)
    return sh.make_config(**base)


def tiny_gqa_config(**kw):
    base = dict(n_heads=4, n_kv_heads=2, qk_norm=1, rope_theta=1e6, norm_eps=1e-6,
                kv_dtype=sh.SH_KV_BF16)
    base.update(kw)
    return tiny_config(**base)


def random_gains(w, seed):
    """Replace unit norm gains with random positive ones (so a dropped gain is visible)."""
    rng = np.random.default_rng(seed)
    for lw in w.layers:
        for k in ("rms_att", "rms_ffn", "q_norm", "k_norm"):
            if k in lw:
                lw[k] = (0.5 + rng.random(lw[k].shape)).astype(np.float32)
    w.rms_final = (0.5 + rng.random(w.rms_final.shape)).astype(np.float32)
    return w


def torch_forward_f64(cfg, w, tokens, alpha=None):
    """Full causal forward in float64 with torch library ops; returns logits [S, V].

    Standard Llama block: pre-RMSNorm attention with interleaved-pair RoPE computed as a
    complex rotation, optional per-head Q/K RMSNorm, grouped K/V heads, SwiGLU FFN,
    residual x + alpha * branch, final RMSNorm and the classifier rows (tied: embedding)."""
    d = torch.float64
    alpha = cfg.residual_scale if alpha is None else alpha
    S = len(tokens)
    H, KVH, hd = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    E = torch.tensor(w.embed, dtype=d)
    tok = torch.tensor(np.asarray(tokens, dtype=np.int64))
    x = E[tok]  # [S, D]
    pos = torch.arange(S, dtype=d)
    inv_freq = torch.tensor([cfg.rope_theta ** (-(2.0 * i) / hd) for i in range(hd // 2)], dtype=d)
    ang = pos[:, None] * inv_freq[None, :]
    rot = torch.polar(torch.ones_like(ang), ang)  # [S, hd/2]

    def rope(t):  # t [S, heads, hd], pairs (2i, 2i+1) as complex numbers
        c = torch.view_as_complex(t.reshape(S, t.shape[1], hd // 2, 2).contiguous())
        return torch.view_as_real(c * rot[:, None, :]).reshape(S, t.shape[1], hd)

    for lw in w.layers:
        T = lambda k: torch.tensor(lw[k], dtype=d)
        xn = F.rms_norm(x, (cfg.dim,), T("rms_att"), eps=cfg.norm_eps)
        q = (xn @ T("wq").T).reshape(S, H, hd)
        k = (xn @ T("wk").T).reshape(S, KVH, hd)
        v = (xn @ T("wv").T).reshape(S, KVH, hd)
        if cfg.qk_norm:
            q = F.rms_norm(q, (hd,), T("q_norm"), eps=cfg.qk_norm_eps)
            k = F.rms_norm(k, (hd,), T("k_norm"), eps=cfg.qk_norm_eps)
        q, k = rope(q), rope(k)
        att = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1),
                                             is_causal=True, enable_gqa=(H != KVH))
        att = att.transpose(0, 1).reshape(S, H * hd)
        x2 = x + alpha * (att @ T("wo").T)
        x2n = F.rms_norm(x2, (cfg.dim,), T("rms_ffn"), eps=cfg.norm_eps)
        g = F.silu(x2n @ T("w1").T) * (x2n @ T("w3").T)
        x = x2 + alpha * (g @ T("w2").T)
    xn = F.rms_norm(x, (cfg.dim,), torch.tensor(w.rms_final, dtype=d), eps=cfg.norm_eps)
    cls = E if w.cls is None else torch.tensor(w.cls, dtype=d)
    return (xn @ cls.T).numpy()


def oracle_stream(ref, prompt, max_new, max_seq):
    """The oracle's greedy Decode (infer.go:136-202 at temperature 0) restated through its
    forwardOne so that every forward's logits are kept: prompt forwards at positions
    0..n-2, then one forward per generated token, first maximum as the next id (argmax,
    infer.go:373-383), stop after EOS=2 or at max_seq tokens. Returns (ids, eos, logits
    [forwards, V]). The prompt must be non-empty and at most max_seq ids long."""
    ref.reset()
    ids = [int(t) for t in prompt]
    assert 0 < len(ids) <= max_seq
    logits = [ref.forward_one(ids[p], p) for p in range(len(ids) - 1)]
    eos = False
    for _ in range(max_new):
        if len(ids) >= max_seq:
            break
        lg = ref.forward_one(ids[-1], len(ids) - 1)
        logits.append(lg)
        ids.append(int(np.argmax(lg)))
        if ids[-1] == 2:
            eos = True
            break
    return np.asarray(ids), eos, np.stack(logits)


def top2_margins(logits):
    """Top-1 minus top-2 logit of each row."""
    part = np.partition(logits, -2, axis=1)
    return part[:, -1] - part[:, -2]


def deepnet_alpha(n_layers):
    """ane/storiesane/residual.go:9: 1/sqrt(2*NLayers), as float32."""
    return float(np.float32(1.0 / math.sqrt(2.0 * n_layers)))


# ---- llama2.c files (ane/stories/weights.go:49-122, tokenizer.go:16-97) --------------------

LLAMA2_ORDER = ("rms_att", "wq", "wk", "wv", "wo", "rms_ffn", "w1", "w2", "w3")


def write_llama2_bin(path, cfg, w, seq_len=None, negative_vocab=False):
    """Writes `w` in the llama2.c checkpoint layout LoadPretrained reads: the seven-int32
    header, embed, then each per-layer tensor for all layers in LLAMA2_ORDER, rms_final."""
    vocab = -cfg.vocab if negative_vocab else cfg.vocab
    hdr = np.array([cfg.dim, cfg.hidden, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, vocab,
                    cfg.max_seq if seq_len is None else seq_len], "<i4")
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        f.write(np.ascontiguousarray(w.embed, "<f4").tobytes())
        for key in LLAMA2_ORDER:
            for lw in w.layers:
                f.write(np.ascontiguousarray(lw[key], "<f4").tobytes())
        f.write(np.ascontiguousarray(w.rms_final, "<f4").tobytes())


def write_tokenizer_bin(path, pieces, max_len=None):
    """tokenizer.bin: int32 max_token_len, then per id (float32 score, int32 len, bytes)."""
    blobs = [p.encode("utf-8") if isinstance(p, str) else p for p in pieces]
    ml = max(1, max(len(b) for b in blobs)) if max_len is None else max_len
    with open(path, "wb") as f:
        f.write(np.array([ml], "<i4").tobytes())
        for i, b in enumerate(blobs):
            f.write(np.array([-float(i)], "<f4").tobytes())
            f.write(np.array([len(b)], "<i4").tobytes())
            f.write(b)


BLZT_LAYER_ORDER = ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "rms_att", "rms_ffn")


def write_blzt(path, cfg, w, version=3, meta=None, opt_value=0.25):
    """A training checkpoint in the layout ane/stories/ckpt.go:13-176 writes: header and meta,
    per layer Wq..W3, RMSAtt, RMSFFN; every layer's Adam M and V (filled with opt_value so a
    reader that does not skip them exactly reads garbage); RMSFinal, its M and V; Embed, its
    M and V. The format has no grouped heads: wk/wv are dim x dim."""
    meta = dict(step=7, total_steps=100, lr=3e-4, loss=2.5, cum_compile=1.25, cum_train=2.5,
                cum_wall=3.75, cum_steps=6, cum_batches=12, adam_t=7) | (meta or {})
    with open(path, "wb") as f:
        f.write(np.array([0x424C5A54, version, meta["step"], meta["total_steps"], cfg.n_layers,
                          cfg.vocab, cfg.dim, cfg.hidden, cfg.n_heads, cfg.max_seq], "<i4").tobytes())
        f.write(np.array([meta["lr"], meta["loss"]], "<f4").tobytes())
        f.write(np.array([meta["cum_compile"], meta["cum_train"], meta["cum_wall"]], "<f8").tobytes())
        f.write(np.array([meta["cum_steps"], meta["cum_batches"], meta["adam_t"], 0, 0, 0], "<i4").tobytes())
        for lw in w.layers:
            for k in BLZT_LAYER_ORDER:
                f.write(np.ascontiguousarray(lw[k], "<f4").tobytes())
        for lw in w.layers:
            for k in BLZT_LAYER_ORDER:
                f.write(np.full(2 * lw[k].size, opt_value, "<f4").tobytes())
        f.write(np.ascontiguousarray(w.rms_final, "<f4").tobytes())
        f.write(np.full(2 * w.rms_final.size, opt_value, "<f4").tobytes())
        f.write(np.ascontiguousarray(w.embed, "<f4").tobytes())
        f.write(np.full(2 * w.embed.size, opt_value, "<f4").tobytes())


def splitmix64_uniforms(seed: int, n: int) -> np.ndarray:
    """The stories-generate sampler's draws: splitmix64 (Vigna's published generator) seeded
    by -seed, each output's top 53 bits as a double in [0, 1)."""
    mask = (1 << 64) - 1
    x = seed & mask
    out = np.empty(n, np.float64)
    for i in range(n):
        x = (x + 0x9E3779B97F4A7C15) & mask
        z = x
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        z ^= z >> 31
        out[i] = (z >> 11) * (1.0 / 9007199254740992.0)
    return out
