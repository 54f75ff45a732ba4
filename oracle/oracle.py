"""ctypes wrapper of oracle/liboracle.so — the CPU restatement of the reference's token loop.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker or the timed CPU baseline. The product never imports it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

OR_KV_F32, OR_KV_F16, OR_KV_BF16 = 0, 1, 2

_F = C.POINTER(C.c_float)
_I32 = C.POINTER(C.c_int32)


class OrConfig(C.Structure):
    _fields_ = [
        ("dim", C.c_int32), ("hidden", C.c_int32), ("n_layers", C.c_int32),
        ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32),
        ("vocab", C.c_int32), ("max_seq", C.c_int32),
        ("rope_theta", C.c_double), ("norm_eps", C.c_double), ("qk_norm_eps", C.c_double),
        ("residual_scale", C.c_float), ("qk_norm", C.c_int32), ("kv_dtype", C.c_int32),
        ("w8a8", C.c_int32),
    ]


class OrLayer(C.Structure):
    _fields_ = [(k, _F) for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3",
                                  "rms_att", "rms_ffn", "q_norm", "k_norm")]


class OrWeights(C.Structure):
    _fields_ = [("layers", C.POINTER(OrLayer)), ("embed", _F), ("rms_final", _F), ("cls", _F)]


class OrTrainLayer(C.Structure):
    _fields_ = [(k, _F) for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "rms_att", "rms_ffn")]


class OrTrainParams(C.Structure):
    _fields_ = [("layers", C.POINTER(OrTrainLayer)), ("embed", _F), ("rms_final", _F)]


class OrTrainHparams(C.Structure):
    _fields_ = [(k, C.c_float) for k in ("lr", "beta1", "beta2", "eps", "weight_decay", "grad_clip",
                                          "loss_scale")]


TRAIN_KEYS = ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "rms_att", "rms_ffn")


_lib = None


def load() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
    lib = C.CDLL(LIB_PATH)
    sig = {
        "or_half_round": (C.c_float, [C.c_float]),
        "or_bf16_round": (C.c_float, [C.c_float]),
        "or_rms_norm_vec": (None, [_F, _F, _F, C.c_int, C.c_double]),
        "or_mat_vec": (None, [_F, _F, _F, C.c_int, C.c_int, C.c_int]),
        "or_silu": (C.c_float, [C.c_float]),
        "or_softmax_prefix": (None, [_F, _F, C.c_int]),
        "or_argmax": (C.c_int32, [_F, C.c_int]),
        "or_rope_tables": (None, [_F, _F, C.c_int, C.c_int, C.c_double]),
        "or_quantize_value": (C.c_int8, [C.c_float]),
        "or_absmax_scale": (C.c_float, [_F, C.c_size_t]),
        "or_quantize_tensor": (None, [_F, C.c_size_t, C.POINTER(C.c_int8), _F]),
        "or_quantize_rows": (None, [_F, C.c_int, C.c_int, C.POINTER(C.c_int8), _F]),
        "or_dequantize_rows": (None, [C.POINTER(C.c_int8), _F, C.c_int, C.c_int, _F]),
        "or_mat_vec_w8a8": (None, [_F, C.POINTER(C.c_int8), _F, _F, C.c_int, C.c_int, C.c_int]),
        "or_decoder_new": (C.c_void_p, [C.POINTER(OrConfig), C.POINTER(OrWeights), C.c_int]),
        "or_decoder_free": (None, [C.c_void_p]),
        "or_decoder_reset": (None, [C.c_void_p]),
        "or_forward_one": (C.c_int, [C.c_void_p, C.c_int, C.c_int, _F]),
        "or_prompt_forward": (C.c_int, [C.c_void_p, _I32, C.c_int, C.c_int, _F]),
        "or_sample_from_logits": (C.c_int, [_F, C.c_int, C.c_float, C.c_double, C.POINTER(C.c_double)]),
        "or_prompt_forward_logits": (C.c_int, [C.c_void_p, _I32, C.c_int, C.c_int, C.c_int, _F]),
        "or_greedy_decode": (C.c_int, [C.c_void_p, _I32, C.c_int, C.c_int, _I32, _I32, _I32, _F]),
        "or_decoder_tap": (_F, [C.c_void_p, C.c_int]),
        "or_embed_lookup_cf": (None, [_F, _F, C.c_int, C.POINTER(C.c_uint16), C.c_int, C.c_int]),
        "or_eval_logits_cf": (None, [C.POINTER(OrConfig), C.POINTER(OrWeights), C.POINTER(C.c_uint16),
                                     C.c_int, _F, C.c_int]),
        "or_eval_logits_cf_ref_threads": (None, [C.POINTER(OrConfig), C.POINTER(OrWeights), C.POINTER(C.c_uint16),
                                     C.c_int, _F, C.c_int]),
        "or_fill_decode_window": (None, [C.POINTER(C.c_uint16), C.c_int, _I32, C.c_int]),
        "or_layer_forward_cf": (None, [C.POINTER(OrConfig), C.POINTER(OrLayer), _F, C.c_int, _F, C.c_int]),
        "or_layer_forward_cf_taps": (None, [C.POINTER(OrConfig), C.POINTER(OrLayer), _F, C.c_int, _F, _F, _F,
                                            C.c_int]),
        "or_rms_norm_final_cf": (None, [_F, _F, _F, C.c_int, C.c_int, C.c_double]),
        "or_matmul_vocab_seq": (None, [_F, _F, _F, C.c_int, C.c_int, C.c_int, C.c_int]),
        "or_linear_cf": (None, [_F, _F, _F, C.c_int, C.c_int, C.c_int, C.c_int]),
        "or_rms_norm_backward_cf": (None, [_F, _F, _F, _F, _F, _F, C.c_int, C.c_int, C.c_int]),
        "or_embed_backward": (None, [_F, _F, C.POINTER(C.c_uint16), C.c_int, C.c_int, C.c_int]),
        "or_cross_entropy_loss": (C.c_float, [_F, _F, C.POINTER(C.c_uint16), C.c_int, C.c_int]),
        "or_train_step": (C.c_float, [C.POINTER(OrConfig), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.POINTER(OrTrainHparams), C.c_int, C.POINTER(C.c_uint16),
                                      C.POINTER(C.c_uint16), C.c_int, C.c_int, C.c_int]),
        "or_train_accumulate": (C.c_float, [C.POINTER(OrConfig), C.c_void_p, C.c_void_p,
                                            C.POINTER(OrTrainHparams), C.POINTER(C.c_uint16),
                                            C.POINTER(C.c_uint16), C.c_int, C.c_int]),
        "or_train_flush": (None, [C.POINTER(OrConfig), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                  C.POINTER(OrTrainHparams), C.c_int, C.c_int]),
        "or_drand48_seed": (C.c_uint64, [C.c_int64]),
        "or_drand48_next": (C.c_double, [C.POINTER(C.c_uint64)]),
        "or_train_window": (C.c_uint64, [C.POINTER(C.c_uint64), C.c_int64, C.c_int]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def fp(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous, (a.dtype, a.flags)
    return a.ctypes.data_as(_F)


def config_from(sh_cfg, w8a8: bool = False, kv_dtype: int | None = None) -> OrConfig:
    """OrConfig from the product's ShConfig (same field meanings)."""
    c = OrConfig()
    for k in ("dim", "hidden", "n_layers", "n_heads", "n_kv_heads", "head_dim", "vocab", "max_seq",
              "rope_theta", "norm_eps", "qk_norm_eps", "residual_scale", "qk_norm"):
        setattr(c, k, getattr(sh_cfg, k))
    c.kv_dtype = sh_cfg.kv_dtype if kv_dtype is None else kv_dtype
    c.w8a8 = int(w8a8)
    return c


class _WeightsHolder:
    """Keeps numpy arrays alive behind an OrWeights struct."""

    def __init__(self, w, n_layers: int):
        self.keep = []
        layers = (OrLayer * n_layers)()
        for l in range(n_layers):
            lw = w.layers[l]
            for k in ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "rms_att", "rms_ffn", "q_norm", "k_norm"):
                a = lw.get(k)
                if a is None:
                    setattr(layers[l], k, None)
                    continue
                a = np.ascontiguousarray(a, np.float32)
                self.keep.append(a)
                setattr(layers[l], k, fp(a))
        self.layers = layers
        emb = np.ascontiguousarray(w.embed, np.float32)
        rmsf = np.ascontiguousarray(w.rms_final, np.float32)
        self.keep += [emb, rmsf]
        cls = None
        if w.cls is not None:
            cls = np.ascontiguousarray(w.cls, np.float32)
            self.keep.append(cls)
        self.s = OrWeights(C.cast(layers, C.POINTER(OrLayer)), fp(emb), fp(rmsf), fp(cls))


class Decoder:
    """or_decoder: the restated stories.Decoder (ane/stories/infer.go)."""

    def __init__(self, cfg: OrConfig, weights, threads: int = 1):
        self.lib = load()
        self.cfg = cfg
        self.w = _WeightsHolder(weights, cfg.n_layers)
        self.h = self.lib.or_decoder_new(C.byref(cfg), C.byref(self.w.s), threads)
        if not self.h:
            raise RuntimeError("or_decoder_new failed")

    def forward_one(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.cfg.vocab, np.float32)
        if self.lib.or_forward_one(self.h, token, pos, fp(out)):
            raise ValueError("or_forward_one: out of range")
        return out

    def prompt_forward(self, tokens, pos0: int = 0) -> np.ndarray:
        """Prompt ids at positions pos0.. in one layer-major pass (equal, bit for bit, to
        forward_one over each); returns the last token's logits."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        out = np.empty(self.cfg.vocab, np.float32)
        if self.lib.or_prompt_forward(self.h, t.ctypes.data_as(_I32), t.size, pos0, fp(out)):
            raise ValueError("or_prompt_forward: out of range")
        return out

    def prompt_forward_logits(self, tokens, first: int, pos0: int = 0) -> np.ndarray:
        """prompt_forward keeping the logits of tokens[first:] ([n - first, V]; each equal, bit
        for bit, to forward_one's at its position): a teacher-forced decode of a given stream."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        out = np.empty((t.size - first, self.cfg.vocab), np.float32)
        if self.lib.or_prompt_forward_logits(self.h, t.ctypes.data_as(_I32), t.size, pos0, first, fp(out)):
            raise ValueError("or_prompt_forward_logits: out of range")
        return out

    def tap(self, which: int, n: int) -> np.ndarray:
        p = self.lib.or_decoder_tap(self.h, which)
        return np.ctypeslib.as_array(p, shape=(n,)).copy()

    def reset(self) -> None:
        self.lib.or_decoder_reset(self.h)

    def greedy_decode(self, prompt, max_new: int):
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32))
        out = np.zeros(self.cfg.max_seq, np.int32)
        margins = np.full(max(max_new, 64), np.nan, np.float32)
        n_out = C.c_int32(0)
        eos = C.c_int32(0)
        pp = p.ctypes.data_as(_I32) if p.size else None
        rc = self.lib.or_greedy_decode(self.h, pp, p.size, max_new, out.ctypes.data_as(_I32),
                                       C.byref(n_out), C.byref(eos), fp(margins))
        if rc:
            raise ValueError("or_greedy_decode: invalid prompt")
        return out[: n_out.value].copy(), bool(eos.value), margins

    def close(self) -> None:
        if self.h:
            self.lib.or_decoder_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def eval_logits_cf(cfg: OrConfig, weights, tokens, threads: int = 1, reference_threading: bool = False) -> np.ndarray:
    """or_eval_logits_cf: engine.go:804-842, channel-first [V, S]. reference_threading: the
    reference's threading (linearCF and attention serial, the vocabulary product over
    `threads`), for timing; the values are the same."""
    t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint16))
    holder = _WeightsHolder(weights, cfg.n_layers)
    out = np.empty((cfg.vocab, t.size), np.float32)
    fn = load().or_eval_logits_cf_ref_threads if reference_threading else load().or_eval_logits_cf
    fn(C.byref(cfg), C.byref(holder.s), t.ctypes.data_as(C.POINTER(C.c_uint16)), t.size, fp(out), threads)
    return out


def layer_forward_cf(cfg: OrConfig, weights, layer: int, x_cf: np.ndarray, threads: int = 1) -> np.ndarray:
    """or_layer_forward_cf: one layer of engine.go:815-838 over channel-first [D, S]."""
    x = np.ascontiguousarray(x_cf, np.float32)
    holder = _WeightsHolder(weights, cfg.n_layers)
    out = np.empty_like(x)
    load().or_layer_forward_cf(C.byref(cfg), C.byref(holder.layers[layer]), fp(x), x.shape[1], fp(out),
                               threads)
    return out


def layer_forward_cf_taps(cfg: OrConfig, weights, layer: int, x_cf: np.ndarray, threads: int = 1):
    """or_layer_forward_cf_taps: the layer's output and its intermediates, channel-first:
    sdpa = concat(x2, q_rope, k_rope, v, att) (stories_dynamic.go:162) and
    ffn = concat(x_next, h1, h3) (stories_dynamic.go:222)."""
    x = np.ascontiguousarray(x_cf, np.float32)
    S = x.shape[1]
    holder = _WeightsHolder(weights, cfg.n_layers)
    qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    out = np.empty_like(x)
    sdpa = np.empty((cfg.dim + 2 * qd + 2 * kvd, S), np.float32)
    ffn = np.empty((cfg.dim + 2 * cfg.hidden, S), np.float32)
    load().or_layer_forward_cf_taps(C.byref(cfg), C.byref(holder.layers[layer]), fp(x), S, fp(out),
                                    fp(sdpa), fp(ffn), threads)
    return out, sdpa, ffn


def rms_norm_final_cf(x_cf: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """or_rms_norm_final_cf: cpu.go:97-111 over channel-first [D, S]."""
    x = np.ascontiguousarray(x_cf, np.float32)
    g = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    load().or_rms_norm_final_cf(fp(out), fp(x), fp(g), x.shape[0], x.shape[1], eps)
    return out


def matmul_vocab_seq(embed: np.ndarray, x_cf: np.ndarray, threads: int = 1) -> np.ndarray:
    """or_matmul_vocab_seq: cpu.go:276-300, logits [V, S] = embed [V, D] . x [D, S]."""
    e = np.ascontiguousarray(embed, np.float32)
    x = np.ascontiguousarray(x_cf, np.float32)
    out = np.empty((e.shape[0], x.shape[1]), np.float32)
    load().or_matmul_vocab_seq(fp(out), fp(e), fp(x), e.shape[0], e.shape[1], x.shape[1], threads)
    return out


def linear_cf(w: np.ndarray, x_cf: np.ndarray, threads: int = 1) -> np.ndarray:
    """or_linear_cf: forward_common.go:35-46, out [O, S] = W [O, I] . in [I, S]."""
    wt = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x_cf, np.float32)
    out = np.empty((wt.shape[0], x.shape[1]), np.float32)
    load().or_linear_cf(fp(out), fp(wt), fp(x), wt.shape[0], wt.shape[1], x.shape[1], threads)
    return out


class TrainParams:
    """Mutable fp32 training tensors (weights, a gradient set or Adam moments): a list of
    per-layer dicts keyed like TRAIN_KEYS, plus embed and rms_final, behind or_train_params."""

    def __init__(self, layers, embed, rms_final):
        self.layers = [{k: np.ascontiguousarray(l[k], np.float32) for k in TRAIN_KEYS} for l in layers]
        self.embed = np.ascontiguousarray(embed, np.float32)
        self.rms_final = np.ascontiguousarray(rms_final, np.float32)
        self._ls = (OrTrainLayer * len(self.layers))()
        for i, l in enumerate(self.layers):
            for k in TRAIN_KEYS:
                setattr(self._ls[i], k, fp(l[k]))
        self.s = OrTrainParams(C.cast(self._ls, C.POINTER(OrTrainLayer)), fp(self.embed), fp(self.rms_final))

    @classmethod
    def from_weights(cls, w):
        return cls(w.layers, w.embed, w.rms_final)

    @classmethod
    def zeros_like(cls, other):
        return cls([{k: np.zeros_like(l[k]) for k in TRAIN_KEYS} for l in other.layers],
                   np.zeros_like(other.embed), np.zeros_like(other.rms_final))

    def clear(self):
        """All tensors set to zero in place (clearModelGrad, train_full.go:110-119)."""
        for _, a in self.tensors():
            a.fill(0)

    def tensors(self):
        """(name, array) pairs in a fixed order."""
        out = []
        for i, l in enumerate(self.layers):
            out += [(f"layers.{i}.{k}", l[k]) for k in TRAIN_KEYS]
        return out + [("rms_final", self.rms_final), ("embed", self.embed)]


def hparams(lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0, grad_clip=0.0, loss_scale=256.0):
    """Engine defaults (engine.go:160-186)."""
    return OrTrainHparams(lr, beta1, beta2, eps, weight_decay, grad_clip, loss_scale)


def train_step(cfg: OrConfig, params: TrainParams, m: TrainParams, v: TrainParams, grads: TrainParams,
               hp: OrTrainHparams, step_t: int, inp, tgt, apply: bool = True, threads: int = 1) -> float:
    """or_train_step: one Engine.Step body (train_full.go CPU path) on a given window."""
    i = np.ascontiguousarray(np.asarray(inp, dtype=np.uint16))
    t = np.ascontiguousarray(np.asarray(tgt, dtype=np.uint16))
    assert i.size == t.size
    return load().or_train_step(C.byref(cfg), C.byref(params.s), C.byref(m.s), C.byref(v.s), C.byref(grads.s),
                                C.byref(hp), step_t, i.ctypes.data_as(C.POINTER(C.c_uint16)),
                                t.ctypes.data_as(C.POINTER(C.c_uint16)), i.size, int(apply), threads)


def train_accumulate(cfg: OrConfig, params: TrainParams, accum: TrainParams, hp: OrTrainHparams, inp, tgt,
                     threads: int = 1) -> float:
    """or_train_accumulate: backwardAndAccumulate (train_full.go:709-774) on a given window."""
    i = np.ascontiguousarray(np.asarray(inp, dtype=np.uint16))
    t = np.ascontiguousarray(np.asarray(tgt, dtype=np.uint16))
    assert i.size == t.size
    return load().or_train_accumulate(C.byref(cfg), C.byref(params.s), C.byref(accum.s), C.byref(hp),
                                      i.ctypes.data_as(C.POINTER(C.c_uint16)),
                                      t.ctypes.data_as(C.POINTER(C.c_uint16)), i.size, threads)


def train_flush(cfg: OrConfig, params: TrainParams, m: TrainParams, v: TrainParams, accum: TrainParams,
                hp: OrTrainHparams, step_t: int, pending: int) -> None:
    """or_train_flush: flushPending (engine.go:540-565); accum keeps the applied gradients."""
    load().or_train_flush(C.byref(cfg), C.byref(params.s), C.byref(m.s), C.byref(v.s), C.byref(accum.s),
                          C.byref(hp), step_t, pending)


def cross_entropy_loss(logits_cf: np.ndarray, targets):
    """or_cross_entropy_loss: cpu.go:173-253; returns (loss, dlogits)."""
    lg = np.ascontiguousarray(logits_cf, np.float32)
    t = np.ascontiguousarray(np.asarray(targets, dtype=np.uint16))
    d = np.empty_like(lg)
    loss = load().or_cross_entropy_loss(fp(d), fp(lg), t.ctypes.data_as(C.POINTER(C.c_uint16)),
                                        lg.shape[0], lg.shape[1])
    return loss, d


def rms_norm_backward_cf(dy_cf, x_cf, w, rrms):
    """or_rms_norm_backward_cf: rmsnorm.go:32-47; returns (dx [d, s], dw [d])."""
    dy = np.ascontiguousarray(dy_cf, np.float32)
    x = np.ascontiguousarray(x_cf, np.float32)
    g = np.ascontiguousarray(w, np.float32)
    r = np.ascontiguousarray(rrms, np.float32)
    dx = np.empty_like(x)
    dw = np.zeros(x.shape[0], np.float32)
    load().or_rms_norm_backward_cf(fp(dx), fp(dw), fp(dy), fp(x), fp(g), fp(r), x.shape[0], x.shape[1], 1)
    return dx, dw


def embed_backward(dembed: np.ndarray, dx_cf: np.ndarray, tokens) -> None:
    """or_embed_backward: cpu.go:74-95, in place on dembed [V, D]."""
    assert dembed.dtype == np.float32 and dembed.flags.c_contiguous
    x = np.ascontiguousarray(dx_cf, np.float32)
    t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint16))
    load().or_embed_backward(fp(dembed), fp(x), t.ctypes.data_as(C.POINTER(C.c_uint16)),
                             dembed.shape[0], dembed.shape[1], x.shape[1])


def sample_from_logits(logits, temperature: float, u: float):
    """or_sample_from_logits: sampleFromLogits (infer.go:347-371) with the draw u given;
    returns (index, slack), slack = the draw's distance from its CDF interval's ends / total."""
    lg = np.ascontiguousarray(np.asarray(logits, dtype=np.float32))
    slack = C.c_double(0)
    i = load().or_sample_from_logits(lg.ctypes.data_as(_F), lg.size, temperature, u, C.byref(slack))
    return int(i), float(slack.value)


def fill_decode_window(seq: int, tokens) -> np.ndarray:
    """or_fill_decode_window: decode.go:83-94, the last `seq` ids left-padded with BOS."""
    t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
    out = np.empty(seq, np.uint16)
    load().or_fill_decode_window(out.ctypes.data_as(C.POINTER(C.c_uint16)), seq,
                                 t.ctypes.data_as(C.POINTER(C.c_int32)), t.size)
    return out


def quantize_rows(src: np.ndarray):
    a = np.ascontiguousarray(src, np.float32)
    rows, cols = a.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    load().or_quantize_rows(fp(a), rows, cols, q.ctypes.data_as(C.POINTER(C.c_int8)), fp(s))
    return q, s


def mat_vec_w8a8(wq: np.ndarray, wscale: np.ndarray, x: np.ndarray, threads: int = 1) -> np.ndarray:
    """or_mat_vec_w8a8: x quantized per tensor, exact int32 dot per row, (float)acc * (s_w * s_a)."""
    q = np.ascontiguousarray(wq, np.int8)
    rows, cols = q.shape
    xx = np.ascontiguousarray(x, np.float32)
    assert xx.size == cols
    out = np.empty(rows, np.float32)
    load().or_mat_vec_w8a8(fp(out), q.ctypes.data_as(C.POINTER(C.c_int8)),
                           fp(np.ascontiguousarray(wscale, np.float32)), fp(xx), rows, cols, threads)
    return out


def quantize_tensor(src: np.ndarray):
    a = np.ascontiguousarray(src, np.float32)
    q = np.empty(a.shape, np.int8)
    s = C.c_float(0)
    load().or_quantize_tensor(fp(a.reshape(-1)), a.size, q.ctypes.data_as(C.POINTER(C.c_int8)), C.byref(s))
    return q, np.float32(s.value)


def dequantize_rows(q: np.ndarray, scales: np.ndarray) -> np.ndarray:
    qq = np.ascontiguousarray(q, np.int8)
    rows, cols = qq.shape
    out = np.empty((rows, cols), np.float32)
    load().or_dequantize_rows(qq.ctypes.data_as(C.POINTER(C.c_int8)), fp(np.ascontiguousarray(scales, np.float32)),
                              rows, cols, fp(out))
    return out
