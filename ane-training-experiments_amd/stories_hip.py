"""ctypes binding of libstories_hip.so (declared in include/stories_hip.h).

Python-side mirror of the reference's decode API for tests, the smoke check and the
benchmark. It mirrors ane/stories (NewDecoder / EvalNextLogits / Decode / ResetCache,
ane/stories/infer.go:61-202) and ane/storiesane (EvalLogits, engine.go:363-376) on top of the
C ABI. There is no fallback: if the shared library is missing, importing `load()` raises.

Synthetic weights (the N(0, std) configurations) come from the library's own deterministic
generator, `sh_synth_normal`, keyed by (seed, tensor id):
    embedding 1, untied classifier 2,
    layer l: 16*(l+1) + {0: wq, 1: wk, 2: wv, 3: wo, 4: w1, 5: w2, 6: w3}.
RMSNorm and QK-norm gains are 1, as in stories.RandomInit (ane/stories/weights.go:142-149).
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libstories_hip.so")

SH_DTYPE_F16 = 1
SH_DTYPE_BF16 = 2
SH_DTYPE_W8A8 = 3
SH_KV_F32 = 0
SH_KV_F16 = 1
SH_KV_BF16 = 2
SH_TAP_X, SH_TAP_QKV, SH_TAP_ATT, SH_TAP_GATE, SH_TAP_X2 = 0, 1, 4, 5, 6
SH_DEBUG_FAIL_NEXT_LAUNCH, SH_DEBUG_PROMPT_PREFILL = 1, 2

BOS = 1
EOS = 2


class ShConfig(C.Structure):
    _fields_ = [
        ("dim", C.c_int32),
        ("hidden", C.c_int32),
        ("n_layers", C.c_int32),
        ("n_heads", C.c_int32),
        ("n_kv_heads", C.c_int32),
        ("head_dim", C.c_int32),
        ("vocab", C.c_int32),
        ("max_seq", C.c_int32),
        ("rope_theta", C.c_double),
        ("norm_eps", C.c_double),
        ("qk_norm_eps", C.c_double),
        ("residual_scale", C.c_float),
        ("qk_norm", C.c_int32),
        ("tied_embed", C.c_int32),
        ("kv_dtype", C.c_int32),
        ("max_batch", C.c_int32),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}

    @property
    def qdim(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kvdim(self) -> int:
        return self.n_kv_heads * self.head_dim


class ShTiming(C.Structure):
    _fields_ = [
        ("gpu_ms", C.c_double),
        ("forwards", C.c_int64),
        ("tokens_out", C.c_int64),
        ("bytes_per_forward_mean", C.c_double),
        ("persistent", C.c_int32),
        ("grid", C.c_int32),
        ("prefill_ms", C.c_double),
    ]


class ShError(RuntimeError):
    pass


_F = C.POINTER(C.c_float)
_I32 = C.POINTER(C.c_int32)
_lib = None

# every entry point of include/stories_hip.h with its ctypes signature
SIGNATURES = {
    "sh_init": (C.c_int, [C.c_int32]),
    "sh_window_greedy_decode": (C.c_int, [C.c_void_p, C.POINTER(C.c_int32), C.c_int32, C.c_int32, C.c_int32,
                                          C.POINTER(C.c_int32), C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    "sh_batch_greedy_decode": (C.c_int, [C.c_void_p, C.POINTER(C.c_int32), C.c_int32, C.c_int32, C.c_int32,
                                         C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    "sh_batch_greedy_decode_logits": (C.c_int, [C.c_void_p, C.POINTER(C.c_int32), C.c_int32, C.c_int32,
                                                C.c_int32, C.POINTER(C.c_int32), C.POINTER(C.c_int32),
                                                C.POINTER(C.c_int32), C.c_int32, C.POINTER(C.c_float)]),
    "sh_decode_tap": (C.c_int, [C.c_void_p, C.c_int32, C.POINTER(C.c_float), C.c_int32]),
    "sh_copy_calibrate": (C.c_int, [C.c_size_t, C.c_int32, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "sh_read_calibrate": (C.c_int, [C.c_size_t, C.c_int32, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "sh_last_error": (C.c_size_t, [C.c_char_p, C.c_size_t]),
    "sh_config_stories110m": (C.c_int, [C.POINTER(ShConfig)]),
    "sh_config_qwen3_06b": (C.c_int, [C.POINTER(ShConfig)]),
    "sh_model_create": (C.c_void_p, [C.POINTER(ShConfig), C.c_int32]),
    "sh_model_upload_layer": (C.c_int, [C.c_void_p, C.c_int32] + [_F] * 11),
    "sh_model_upload_globals": (C.c_int, [C.c_void_p, _F, _F, _F]),
    "sh_reset_cache": (C.c_int, [C.c_void_p]),
    "sh_decode_step": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, _F, _I32]),
    "sh_greedy_decode": (C.c_int, [C.c_void_p, _I32, C.c_int32, C.c_int32, _I32, _I32, _I32]),
    "sh_prefill_logits": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint16), C.c_int32, _F]),
    "sh_stats": (C.c_int, [C.c_void_p, C.POINTER(ShTiming)]),
    "sh_model_describe": (C.c_size_t, [C.c_void_p, C.c_char_p, C.c_size_t]),
    "sh_trace_forward": (C.c_int, [C.c_void_p, C.c_int32]),
    "sh_debug_option": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32]),
    "sh_trace_read": (C.c_int, [C.c_void_p, C.POINTER(C.c_int64), C.c_int32, _I32, C.POINTER(C.c_double)]),
    "sh_model_destroy": (None, [C.c_void_p]),
    "sh_quantize_i8": (C.c_int, [_F, C.c_int32, C.c_int32, C.POINTER(C.c_int8), _F, C.c_int32]),
    "sh_dequantize_i8": (C.c_int, [C.POINTER(C.c_int8), _F, C.c_int32, C.c_int32, C.c_int32, _F]),
    "sh_synth_normal": (C.c_int, [_F, C.c_size_t, C.c_uint64, C.c_uint64, C.c_float]),
    "sh_synth_tokens": (C.c_int, [_I32, C.c_size_t, C.c_uint64, C.c_int32]),
    "sh_round_dtype": (C.c_int, [_F, C.c_size_t, C.c_int32]),
    "sh_layer_forward_cf": (C.c_int, [C.c_void_p, C.c_int32, _F, C.c_int32, _F]),
    "sh_model_read_weights": (C.c_int, [C.c_void_p, C.c_int32, C.c_char_p, C.c_void_p, C.c_size_t]),
    "sh_layer_forward_cf_taps": (C.c_int, [C.c_void_p, C.c_int32, _F, C.c_int32, _F, _F, _F]),
    "sh_rms_final_cf": (C.c_int, [C.c_void_p, _F, C.c_int32, _F]),
    "sh_classifier_cf": (C.c_int, [C.c_void_p, _F, C.c_int32, _F]),
    "sh_matmul_vocab_seq": (C.c_int, [_F, _F, C.c_int32, C.c_int32, C.c_int32, _F]),
    "sh_conv_create": (C.c_void_p, [_F, C.c_int32, C.c_int32]),
    "sh_conv_eval": (C.c_int, [C.c_void_p, _F, C.c_int32, _F]),
    "sh_conv_destroy": (None, [C.c_void_p]),
    "sh_conv_eval_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p]),
    "sh_trainer_create": (C.c_void_p, [C.POINTER(ShConfig), C.c_void_p]),
    "sh_trainer_upload_layer": (C.c_int, [C.c_void_p, C.c_int32] + [_F] * 9),
    "sh_trainer_upload_globals": (C.c_int, [C.c_void_p, _F, _F]),
    "sh_trainer_set_tokens": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint16), C.c_int64]),
    "sh_trainer_step": (C.c_int, [C.c_void_p, _F]),
    "sh_trainer_step_window": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint16), C.POINTER(C.c_uint16), _F]),
    "sh_trainer_flush": (C.c_int, [C.c_void_p]),
    "sh_trainer_read": (C.c_int, [C.c_void_p, C.c_int32, C.c_char_p, _F, C.c_size_t]),
    "sh_trainer_state": (C.c_int, [C.c_void_p, C.c_void_p]),
    "sh_trainer_destroy": (None, [C.c_void_p]),
}


def load(path: str = LIB_PATH) -> C.CDLL:
    """Loads the HIP library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ShError(f"{path} is missing: build it with __graft_entry__.build()")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    lib = load()
    buf = C.create_string_buffer(4096)
    lib.sh_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ShError(f"{what}: {last_error()}")


def _fp(a: np.ndarray | None):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def init(device: int = 0) -> None:
    _check(load().sh_init(device), "sh_init")


def stories110m_config() -> ShConfig:
    c = ShConfig()
    _check(load().sh_config_stories110m(C.byref(c)), "sh_config_stories110m")
    return c


def qwen3_06b_config() -> ShConfig:
    c = ShConfig()
    _check(load().sh_config_qwen3_06b(C.byref(c)), "sh_config_qwen3_06b")
    return c


def make_config(**kw) -> ShConfig:
    """A config from keyword fields; unspecified fields take the Stories110M defaults."""
    c = stories110m_config()
    for k, v in kw.items():
        if not hasattr(c, k):
            raise KeyError(k)
        setattr(c, k, v)
    return c


# ---- synthetic inputs ------------------------------------------------------------------

def synth_normal(n: int, seed: int, tensor_id: int, std: float) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _check(load().sh_synth_normal(_fp(out), n, seed, tensor_id, std), "sh_synth_normal")
    return out


def synth_tokens(n: int, seed: int, vocab: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    _check(load().sh_synth_tokens(out.ctypes.data_as(_I32), n, seed, vocab), "sh_synth_tokens")
    return out


def round_dtype(a: np.ndarray, dtype: int) -> np.ndarray:
    """Rounds a copy of fp32 `a` to the values `dtype` stores (round to nearest even)."""
    out = np.ascontiguousarray(a, dtype=np.float32).copy()
    _check(load().sh_round_dtype(_fp(out), out.size, dtype), "sh_round_dtype")
    return out


LAYER_KEYS = ("wq", "wk", "wv", "wo", "w1", "w2", "w3")


def layer_shapes(cfg: ShConfig) -> dict:
    D, F, Q, KV = cfg.dim, cfg.hidden, cfg.qdim, cfg.kvdim
    return {"wq": (Q, D), "wk": (KV, D), "wv": (KV, D), "wo": (D, Q),
            "w1": (F, D), "w2": (D, F), "w3": (F, D)}


@dataclass
class Weights:
    """Host fp32 weights in the reference's layout (ane/stories/weights.go:13-24)."""
    layers: list
    embed: np.ndarray
    rms_final: np.ndarray
    cls: np.ndarray | None  # None when tied to embed

    def rounded(self, dtype: int) -> "Weights":
        """The values the device computes with. fp16 / bf16: every matrix rounded (norm
        gains stay fp32). W8A8: matrices stay fp32 (a CPU check quantizes them itself), the
        lookup table is fp16, and the classifier is quantized from the fp32 rows, so the
        tied classifier is returned explicitly as `cls`."""
        if dtype == SH_DTYPE_W8A8:
            cls = self.cls if self.cls is not None else self.embed
            return Weights(self.layers, round_dtype(self.embed, SH_DTYPE_F16), self.rms_final, cls)
        if dtype not in (SH_DTYPE_F16, SH_DTYPE_BF16):
            return self
        layers = []
        for lw in self.layers:
            d = dict(lw)
            for k in LAYER_KEYS:
                d[k] = round_dtype(lw[k], dtype)
            layers.append(d)
        embed = round_dtype(self.embed, dtype)
        cls = None if self.cls is None else round_dtype(self.cls, dtype)
        return Weights(layers, embed, self.rms_final, cls)


def synth_weights(cfg: ShConfig, seed: int, std: float = 0.02) -> Weights:
    """N(0, std) matrices and unit norm gains for `cfg` (see the module docstring)."""
    shapes = layer_shapes(cfg)
    layers = []
    for l in range(cfg.n_layers):
        lw = {}
        for j, k in enumerate(LAYER_KEYS):
            r, c = shapes[k]
            lw[k] = synth_normal(r * c, seed, 16 * (l + 1) + j, std).reshape(r, c)
        lw["rms_att"] = np.ones(cfg.dim, np.float32)
        lw["rms_ffn"] = np.ones(cfg.dim, np.float32)
        if cfg.qk_norm:
            lw["q_norm"] = np.ones(cfg.head_dim, np.float32)
            lw["k_norm"] = np.ones(cfg.head_dim, np.float32)
        layers.append(lw)
    embed = synth_normal(cfg.vocab * cfg.dim, seed, 1, std).reshape(cfg.vocab, cfg.dim)
    cls = None
    if not cfg.tied_embed:
        cls = synth_normal(cfg.vocab * cfg.dim, seed, 2, std).reshape(cfg.vocab, cfg.dim)
    return Weights(layers, embed, np.ones(cfg.dim, np.float32), cls)


# ---- model -----------------------------------------------------------------------------

class Model:
    """A device-resident model: stories.Decoder (infer.go:30-59) + storiesane.Engine
    (engine.go:67-146) surface over the C ABI."""

    def __init__(self, cfg: ShConfig, dtype: int):
        self.lib = load()
        self.cfg = cfg
        self.dtype = dtype
        self.h = self.lib.sh_model_create(C.byref(cfg), dtype)
        if not self.h:
            raise ShError(f"sh_model_create: {last_error()}")

    def _upload_layer(self, l: int, lw: dict) -> None:
        arrs = [np.ascontiguousarray(lw[k], np.float32) for k in LAYER_KEYS]
        arrs += [np.ascontiguousarray(lw["rms_att"], np.float32),
                 np.ascontiguousarray(lw["rms_ffn"], np.float32)]
        qn = lw.get("q_norm")
        kn = lw.get("k_norm")
        qn = None if qn is None else np.ascontiguousarray(qn, np.float32)
        kn = None if kn is None else np.ascontiguousarray(kn, np.float32)
        _check(self.lib.sh_model_upload_layer(self.h, l, *[_fp(a) for a in arrs], _fp(qn), _fp(kn)),
               f"sh_model_upload_layer({l})")

    def upload(self, w: Weights) -> None:
        for l, lw in enumerate(w.layers):
            self._upload_layer(l, lw)
        embed = np.ascontiguousarray(w.embed, np.float32)
        cls = None if w.cls is None else np.ascontiguousarray(w.cls, np.float32)
        _check(self.lib.sh_model_upload_globals(self.h, _fp(embed), _fp(np.ascontiguousarray(w.rms_final, np.float32)), _fp(cls)),
               "sh_model_upload_globals")

    def reset_cache(self) -> None:
        _check(self.lib.sh_reset_cache(self.h), "sh_reset_cache")

    def eval_next_logits(self, token: int, pos: int, want_logits: bool = True):
        """(*Decoder).EvalNextLogits (infer.go:72-77): returns (logits or None, argmax)."""
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        am = C.c_int32(0)
        _check(self.lib.sh_decode_step(self.h, token, pos, _fp(logits), C.byref(am)), "sh_decode_step")
        return logits, am.value

    def greedy_decode(self, prompt, max_new: int):
        """(*Decoder).Decode with Temperature 0 (infer.go:136-202).
        Returns (tokens, prompt_length, stopped_on_eos)."""
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32))
        out = np.zeros(self.cfg.max_seq, np.int32)
        n_out = C.c_int32(0)
        eos = C.c_int32(0)
        pp = p.ctypes.data_as(_I32) if p.size else None
        _check(self.lib.sh_greedy_decode(self.h, pp, p.size, max_new, out.ctypes.data_as(_I32),
                                         C.byref(n_out), C.byref(eos)), "sh_greedy_decode")
        plen = min(max(p.size, 1), self.cfg.max_seq)
        return out[: n_out.value].copy(), plen, bool(eos.value)

    def eval_logits(self, tokens) -> np.ndarray:
        """(*Engine).EvalLogits (engine.go:363-376): channel-first [V, S] logits."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint16))
        out = np.empty((self.cfg.vocab, t.size), np.float32)
        _check(self.lib.sh_prefill_logits(self.h, t.ctypes.data_as(C.POINTER(C.c_uint16)), t.size, _fp(out)),
               "sh_prefill_logits")
        return out

    def read_weights(self, layer: int, name: str) -> np.ndarray:
        """sh_model_read_weights: a tensor as stored on the device: uint16 bits (fp16 / bf16),
        int8 rows (W8A8) or, for "<name>.scale", float32 row scales."""
        c = self.cfg
        shapes = {"wq": (c.qdim, c.dim), "wk": (c.kvdim, c.dim), "wv": (c.kvdim, c.dim),
                  "wo": (c.dim, c.qdim), "w1": (c.hidden, c.dim), "w3": (c.hidden, c.dim),
                  "w2": (c.dim, c.hidden), "embed": (c.vocab, c.dim), "cls": (c.vocab, c.dim)}
        base = name[:-6] if name.endswith(".scale") else name
        rows, cols = shapes[base]
        if name.endswith(".scale"):
            out = np.empty(rows, np.float32)
        elif self.dtype == SH_DTYPE_W8A8 and base != "embed":
            out = np.empty((rows, cols), np.int8)
        else:
            out = np.empty((rows, cols), np.uint16)
        _check(self.lib.sh_model_read_weights(self.h, layer, name.encode(), out.ctypes.data_as(C.c_void_p),
                                              out.nbytes), "sh_model_read_weights")
        return out

    def layer_forward_cf(self, layer: int, x_cf: np.ndarray) -> np.ndarray:
        """One layer over channel-first [dim, seq] (the storiesane layerForward.run seam)."""
        x = np.ascontiguousarray(x_cf, np.float32)
        out = np.empty_like(x)
        _check(self.lib.sh_layer_forward_cf(self.h, layer, _fp(x), x.shape[1], _fp(out)), "sh_layer_forward_cf")
        return out

    def layer_forward_cf_taps(self, layer: int, x_cf: np.ndarray):
        """sh_layer_forward_cf_taps: (out, sdpa, ffn) channel-first, sdpa = concat(x2, q_rope,
        k_rope, v, att) and ffn = concat(x_next, h1, h3) (stories_dynamic.go:162, :222)."""
        x = np.ascontiguousarray(x_cf, np.float32)
        S = x.shape[1]
        c = self.cfg
        out = np.empty_like(x)
        sdpa = np.empty((c.dim + 2 * c.qdim + 2 * c.kvdim, S), np.float32)
        ffn = np.empty((c.dim + 2 * c.hidden, S), np.float32)
        _check(self.lib.sh_layer_forward_cf_taps(self.h, layer, _fp(x), S, _fp(out), _fp(sdpa), _fp(ffn)),
               "sh_layer_forward_cf_taps")
        return out, sdpa, ffn

    def rms_final_cf(self, x_cf: np.ndarray) -> np.ndarray:
        """The final RMSNorm over channel-first [dim, seq] (offload.runRMSForward)."""
        x = np.ascontiguousarray(x_cf, np.float32)
        out = np.empty_like(x)
        _check(self.lib.sh_rms_final_cf(self.h, _fp(x), x.shape[1], _fp(out)), "sh_rms_final_cf")
        return out

    def classifier_cf(self, xnorm_cf: np.ndarray) -> np.ndarray:
        """logits [vocab, seq] from channel-first [dim, seq] (offload.runClassifierForward)."""
        x = np.ascontiguousarray(xnorm_cf, np.float32)
        out = np.empty((self.cfg.vocab, x.shape[1]), np.float32)
        _check(self.lib.sh_classifier_cf(self.h, _fp(x), x.shape[1], _fp(out)), "sh_classifier_cf")
        return out

    def tap(self, which: int) -> np.ndarray:
        """sh_decode_tap: an intermediate vector of the last layer of the last forward."""
        n = {SH_TAP_X: self.cfg.dim, SH_TAP_QKV: self.cfg.qdim + 2 * self.cfg.kvdim,
             SH_TAP_ATT: self.cfg.qdim, SH_TAP_GATE: self.cfg.hidden, SH_TAP_X2: self.cfg.dim}[which]
        out = np.empty(n, np.float32)
        _check(self.lib.sh_decode_tap(self.h, which, _fp(out), n), "sh_decode_tap")
        return out

    def window_greedy_decode(self, prompt, seq: int, max_new: int):
        """(*Engine).Decode with Temperature 0 (decode.go:18-94): (tokens, prompt_len, eos)."""
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32))
        plen = max(1, min(p.size, seq))
        out = np.zeros(plen + (max_new if max_new > 0 else 64), np.int32)
        n, eos = C.c_int32(0), C.c_int32(0)
        _check(self.lib.sh_window_greedy_decode(self.h, p.ctypes.data_as(_I32) if p.size else None, p.size,
                                                 seq, max_new, out.ctypes.data_as(_I32), C.byref(n),
                                                 C.byref(eos)), "sh_window_greedy_decode")
        return out[:n.value].copy(), plen, bool(eos.value)

    def batch_greedy_decode(self, prompts, max_new: int):
        """sh_batch_greedy_decode: list of token arrays (prompt + generated, EOS-truncated)."""
        p = np.ascontiguousarray(np.asarray(prompts, dtype=np.int32))
        if p.ndim != 2:
            raise ValueError("prompts must be a 2-D array [n_seqs, prompt_len]")
        n, plen = p.shape
        stride = plen + (max_new if max_new > 0 else 64)
        out = np.zeros((n, stride), np.int32)
        cnt = np.zeros(n, np.int32)
        _check(self.lib.sh_batch_greedy_decode(self.h, p.ctypes.data_as(_I32), n, plen, max_new,
                                                out.ctypes.data_as(_I32), cnt.ctypes.data_as(_I32)),
               "sh_batch_greedy_decode")
        return [out[i, :cnt[i]].copy() for i in range(n)]

    def batch_greedy_decode_logits(self, prompts, max_new: int, rows):
        """sh_batch_greedy_decode_logits: (token arrays as batch_greedy_decode, logits
        [steps, len(rows), V] of the chosen sequences at every step)."""
        p = np.ascontiguousarray(np.asarray(prompts, dtype=np.int32))
        if p.ndim != 2:
            raise ValueError("prompts must be a 2-D array [n_seqs, prompt_len]")
        n, plen = p.shape
        mn = max_new if max_new > 0 else 64
        steps = min(mn, self.cfg.max_seq - plen)
        r = np.ascontiguousarray(np.asarray(rows, dtype=np.int32))
        out = np.zeros((n, plen + mn), np.int32)
        cnt = np.zeros(n, np.int32)
        lg = np.zeros((max(steps, 1), r.size, self.cfg.vocab), np.float32)
        _check(self.lib.sh_batch_greedy_decode_logits(self.h, p.ctypes.data_as(_I32), n, plen, max_new,
                                                       out.ctypes.data_as(_I32), cnt.ctypes.data_as(_I32),
                                                       r.ctypes.data_as(_I32), r.size, _fp(lg)),
               "sh_batch_greedy_decode_logits")
        return [out[i, :cnt[i]].copy() for i in range(n)], lg[:steps]

    def debug_fail_next_launch(self, mode: int) -> None:
        """Testing aid: the next persistent launch ends at once, as a residency failure (2) or
        a hand-over timeout with every workgroup running (1); 0 disarms."""
        _check(self.lib.sh_debug_option(self.h, SH_DEBUG_FAIL_NEXT_LAUNCH, mode), "sh_debug_option")

    def set_prompt_prefill(self, on: bool) -> None:
        """Testing aid: False feeds a greedy decode's prompt through the token loop."""
        _check(self.lib.sh_debug_option(self.h, SH_DEBUG_PROMPT_PREFILL, int(bool(on))), "sh_debug_option")

    def trace_forward(self, forward: int) -> None:
        _check(self.lib.sh_trace_forward(self.h, forward), "sh_trace_forward")

    def _trace_raw(self):
        L = self.cfg.n_layers
        n = self.stats()["grid"] * 2 * (5 * L + 3)
        buf = np.zeros(n, np.int64)
        cnt = C.c_int32(0)
        rate = C.c_double(0)
        _check(self.lib.sh_trace_read(self.h, buf.ctypes.data_as(C.POINTER(C.c_int64)), n, C.byref(cnt),
                                      C.byref(rate)), "sh_trace_read")
        t = buf[:cnt.value].reshape(-1, 2, 5 * L + 3).astype(np.float64)
        return t, rate.value

    def trace_stamps(self) -> np.ndarray:
        """Stage-end timestamps (us, from the earliest forward start) of the traced forward:
        [grid, 5 * n_layers + 3], one row per workgroup."""
        t, rate = self._trace_raw()
        return (t[:, 0] - t[:, 0, 0].min()) * 1e6 / rate

    def trace_inputs(self) -> np.ndarray:
        """Input-ready timestamps (us, same origin as trace_stamps): column j is when the
        workgroup had the whole input of the stage whose end is column j of trace_stamps
        (NaN where the workgroup had no input to wait for in that stage)."""
        t, rate = self._trace_raw()
        out = (t[:, 1] - t[:, 0, 0].min()) * 1e6 / rate
        out[t[:, 1] == 0] = np.nan
        return out

    def trace_read(self) -> dict:
        """Critical-path stage durations (us) of the traced forward, summed over layers: a
        stage ends when its last workgroup stamps it."""
        L = self.cfg.n_layers
        ends = self.trace_stamps().max(axis=0)
        d = np.diff(ends)
        names = ["qkv", "attn", "wo", "w13", "w2"]
        out = {k: float(d[j:5 * L:5].sum()) for j, k in enumerate(names)}
        out["classifier"] = float(d[5 * L])
        out["argmax"] = float(d[5 * L + 1])
        out["total"] = float(ends[-1] - ends[0])
        return out

    def describe(self) -> str:
        buf = C.create_string_buffer(1024)
        self.lib.sh_model_describe(self.h, buf, len(buf))
        return buf.value.decode(errors="replace")

    def stats(self) -> dict:
        t = ShTiming()
        _check(self.lib.sh_stats(self.h, C.byref(t)), "sh_stats")
        return {"gpu_ms": t.gpu_ms, "forwards": t.forwards, "tokens_out": t.tokens_out,
                "bytes_per_forward_mean": t.bytes_per_forward_mean,
                "persistent": bool(t.persistent), "grid": t.grid, "prefill_ms": t.prefill_ms}

    def close(self) -> None:
        if self.h:
            self.lib.sh_model_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def copy_calibrate(nbytes: int, reps: int = 10):
    """sh_copy_calibrate: (ms per copy, GB/s) of the plain copy kernel over nbytes."""
    ms, gbps = C.c_double(0), C.c_double(0)
    _check(load().sh_copy_calibrate(nbytes, reps, C.byref(ms), C.byref(gbps)), "sh_copy_calibrate")
    return ms.value, gbps.value


def read_calibrate(nbytes: int, reps: int = 10):
    """sh_read_calibrate: (ms per pass, GB/s) of the plain read-only kernel over nbytes."""
    ms, gbps = C.c_double(0), C.c_double(0)
    _check(load().sh_read_calibrate(nbytes, reps, C.byref(ms), C.byref(gbps)), "sh_read_calibrate")
    return ms.value, gbps.value


def matmul_vocab_seq(embed: np.ndarray, x_cf: np.ndarray) -> np.ndarray:
    """logits [vocab, seq] = embed [vocab, dim] . x [dim, seq] (matMulVocabSeqAccelerate)."""
    lib = load()
    e = np.ascontiguousarray(embed, np.float32)
    x = np.ascontiguousarray(x_cf, np.float32)
    out = np.empty((e.shape[0], x.shape[1]), np.float32)
    _check(lib.sh_matmul_vocab_seq(_fp(e), _fp(x), e.shape[0], e.shape[1], x.shape[1], _fp(out)),
           "sh_matmul_vocab_seq")
    return out


class Conv:
    """A compiled 1x1 conv (model.Kernel) for forward.ConvEval: y [s, out] = x [s, in] . w^T."""

    def __init__(self, w: np.ndarray):
        self.lib = load()
        self.w = np.ascontiguousarray(w, np.float32)
        self.h = self.lib.sh_conv_create(_fp(self.w), self.w.shape[0], self.w.shape[1])
        if not self.h:
            raise ShError(f"sh_conv_create: {last_error()}")

    def eval(self, x: np.ndarray) -> np.ndarray:
        a = np.ascontiguousarray(x, np.float32).reshape(-1, self.w.shape[1])
        out = np.empty((a.shape[0], self.w.shape[0]), np.float32)
        _check(self.lib.sh_conv_eval(self.h, _fp(a), a.shape[0], _fp(out)), "sh_conv_eval")
        return out

    def close(self) -> None:
        if self.h:
            self.lib.sh_conv_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class TrainOptions(C.Structure):
    """sh_train_options (storiesane.Options); zero fields take the engine's defaults."""
    _fields_ = [("seq", C.c_int32), ("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float),
                ("eps", C.c_float), ("weight_decay", C.c_float), ("grad_clip", C.c_float),
                ("loss_scale", C.c_float), ("seed", C.c_int64), ("accum_steps", C.c_int32)]


class TrainState(C.Structure):
    _fields_ = [("token_pos", C.c_uint64), ("last_loss", C.c_float), ("cum_steps", C.c_uint32),
                ("adam_t", C.c_uint32), ("last_step_ms", C.c_double), ("cum_batches", C.c_uint32),
                ("pending_steps", C.c_uint32)]


SH_TRAIN_PARAMS, SH_TRAIN_GRADS, SH_TRAIN_ADAM_M, SH_TRAIN_ADAM_V = 0, 1, 2, 3
TRAIN_KEYS = ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "rms_att", "rms_ffn")


class Trainer:
    """The storiesane training engine (Engine.Step) on the device, fp32."""

    def __init__(self, cfg: ShConfig, **opts):
        self.lib = load()
        self.cfg = cfg
        self.opt = TrainOptions(**opts)
        self.h = self.lib.sh_trainer_create(C.byref(cfg), C.byref(self.opt))
        if not self.h:
            raise ShError(f"sh_trainer_create: {last_error()}")
        self.seq = self.opt.seq if self.opt.seq > 0 else 256

    def upload(self, w: Weights) -> None:
        for l, lw in enumerate(w.layers):
            arrs = [np.ascontiguousarray(lw[k], np.float32) for k in TRAIN_KEYS]
            _check(self.lib.sh_trainer_upload_layer(self.h, l, *[_fp(a) for a in arrs]),
                   f"sh_trainer_upload_layer({l})")
        e = np.ascontiguousarray(w.embed, np.float32)
        r = np.ascontiguousarray(w.rms_final, np.float32)
        _check(self.lib.sh_trainer_upload_globals(self.h, _fp(e), _fp(r)), "sh_trainer_upload_globals")

    def set_tokens(self, tokens) -> None:
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint16))
        self._tokens = t
        _check(self.lib.sh_trainer_set_tokens(self.h, t.ctypes.data_as(C.POINTER(C.c_uint16)), t.size),
               "sh_trainer_set_tokens")

    def step(self) -> float:
        loss = C.c_float(0)
        _check(self.lib.sh_trainer_step(self.h, C.byref(loss)), "sh_trainer_step")
        return loss.value

    def step_window(self, inp, tgt) -> float:
        i = np.ascontiguousarray(np.asarray(inp, dtype=np.uint16))
        t = np.ascontiguousarray(np.asarray(tgt, dtype=np.uint16))
        loss = C.c_float(0)
        _check(self.lib.sh_trainer_step_window(self.h, i.ctypes.data_as(C.POINTER(C.c_uint16)),
                                               t.ctypes.data_as(C.POINTER(C.c_uint16)), C.byref(loss)),
               "sh_trainer_step_window")
        return loss.value

    def flush(self) -> None:
        """Engine.Flush: applies pending accumulated gradients (no-op when none are pending)."""
        _check(self.lib.sh_trainer_flush(self.h), "sh_trainer_flush")

    def read(self, which: int, name: str, shape) -> np.ndarray:
        out = np.empty(shape, np.float32)
        _check(self.lib.sh_trainer_read(self.h, which, name.encode(), _fp(out), out.size), "sh_trainer_read")
        return out

    def state(self) -> dict:
        st = TrainState()
        _check(self.lib.sh_trainer_state(self.h, C.byref(st)), "sh_trainer_state")
        return {"token_pos": st.token_pos, "last_loss": st.last_loss, "cum_steps": st.cum_steps,
                "adam_t": st.adam_t, "last_step_ms": st.last_step_ms, "cum_batches": st.cum_batches,
                "pending_steps": st.pending_steps}

    def close(self) -> None:
        if self.h:
            self.lib.sh_trainer_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def quantize_i8(src: np.ndarray, per_row: bool):
    """Device int8 quantizer (bridge/ane_bridge.m:374-399). Returns (q, scales)."""
    a = np.ascontiguousarray(src, np.float32)
    rows, cols = (a.shape if a.ndim == 2 else (1, a.size))
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows if per_row else 1, np.float32)
    _check(load().sh_quantize_i8(_fp(a), rows, cols, q.ctypes.data_as(C.POINTER(C.c_int8)), _fp(s), int(per_row)),
           "sh_quantize_i8")
    return q, s


def dequantize_i8(q: np.ndarray, scales: np.ndarray, per_row: bool) -> np.ndarray:
    qq = np.ascontiguousarray(q, np.int8)
    rows, cols = qq.shape
    out = np.empty((rows, cols), np.float32)
    s = np.ascontiguousarray(scales, np.float32)
    _check(load().sh_dequantize_i8(qq.ctypes.data_as(C.POINTER(C.c_int8)), _fp(s), rows, cols, int(per_row), _fp(out)),
           "sh_dequantize_i8")
    return out
