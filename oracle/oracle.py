"""ctypes wrapper of liboracle.so — the CPU restatement of the reference's
hot-path ops (oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. The product never uses it.
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np

ORACLE_DIR = pathlib.Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_lib = None


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise FileNotFoundError(f"{LIB_PATH} not built (make -C oracle)")
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.oracle_set_workers.restype = ctypes.c_int
    lib.oracle_set_workers.argtypes = [ctypes.c_int]
    lib.oracle_default_workers.restype = ctypes.c_int
    lib.oracle_default_workers.argtypes = []
    lib.oracle_rms_norm_f32.restype = None
    lib.oracle_rms_norm_f32.argtypes = [_P, _P, _P, _I64, _I64, ctypes.c_float]
    lib.oracle_rope_theta_table.restype = None
    lib.oracle_rope_theta_table.argtypes = [ctypes.c_float, ctypes.c_uint32, ctypes.c_uint32, _P]
    lib.oracle_rope_neox_f32.restype = ctypes.c_int
    lib.oracle_rope_neox_f32.argtypes = [_P, _P, _P, _I64, _P, _I64, _I64, _I64]
    lib.oracle_flash_attn_f32.restype = None
    lib.oracle_flash_attn_f32.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64]
    lib.oracle_cpy.restype = ctypes.c_int
    lib.oracle_cpy.argtypes = [_P, _P, ctypes.c_size_t]
    lib.oracle_decode_append_attn_f32.restype = None
    lib.oracle_decode_append_attn_f32.argtypes = [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64]
    _lib = lib
    return lib


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


def set_workers(n: int) -> int:
    """Sets the pool size; returns the number of threads doing work."""
    return load().oracle_set_workers(n)


def default_workers() -> int:
    return load().oracle_default_workers()


def rms_norm(x, w, eps):
    x = _f32(x)
    w = _f32(w)
    out = np.empty_like(x)
    dim = x.shape[-1]
    load().oracle_rms_norm_f32(x.ctypes.data, w.ctypes.data, out.ctypes.data, x.size // dim, dim, eps)
    return out


def rope_theta_table(theta_base: float, head_dim: int, n_ctx: int):
    out = np.empty((n_ctx, head_dim // 2), dtype=np.float32)
    load().oracle_rope_theta_table(theta_base, head_dim, n_ctx, out.ctypes.data)
    return out


def rope_neox(x, pos, theta):
    """x: [n_tokens, n_heads, D]; pos int32 [n_tokens]; theta [n_ctx, D/2]."""
    x = _f32(x)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    theta = _f32(theta)
    out = np.empty_like(x)
    n_tokens, n_heads, D = x.shape
    rc = load().oracle_rope_neox_f32(x.ctypes.data, pos.ctypes.data, theta.ctypes.data,
                                     theta.shape[0], out.ctypes.data, D, n_heads, n_tokens)
    if rc != 0:
        raise ValueError("rope position outside the angle table")
    return out


def flash_attn(q, k, v, n_past: int, n_kv: int | None = None):
    """q [n_q, Hq, D]; k, v [n_kv, Hkv, D] -> out [n_q, Hq, D]."""
    q = _f32(q)
    k = _f32(k)
    v = _f32(v)
    n_q, Hq, D = q.shape
    Hkv = k.shape[1]
    if n_kv is None:
        n_kv = k.shape[0]
    out = np.empty_like(q)
    load().oracle_flash_attn_f32(q.ctypes.data, k.ctypes.data, v.ctypes.data, out.ctypes.data,
                                 D, Hq, n_q, Hkv, n_kv, n_past)
    return out


def cpy(dst, src):
    src = np.ascontiguousarray(src)
    assert dst.flags.c_contiguous and dst.nbytes == src.nbytes
    rc = load().oracle_cpy(dst.ctypes.data, src.ctypes.data, src.nbytes)
    if rc != 0:
        raise ValueError("cpy rejected")


def decode_append_attn(q, k_new, v_new, k_cache, v_cache, n_past: int):
    """In place on k_cache/v_cache [capacity, Hkv, D]; returns out [Hq, D]."""
    q = _f32(q)
    k_new = _f32(k_new)
    v_new = _f32(v_new)
    assert k_cache.dtype == np.float32 and k_cache.flags.c_contiguous
    assert v_cache.dtype == np.float32 and v_cache.flags.c_contiguous
    Hq, D = q.shape[-2], q.shape[-1]
    Hkv = k_cache.shape[1]
    out = np.empty((Hq, D), dtype=np.float32)
    load().oracle_decode_append_attn_f32(q.ctypes.data, k_new.ctypes.data, v_new.ctypes.data,
                                         k_cache.ctypes.data, v_cache.ctypes.data, out.ctypes.data,
                                         D, Hq, Hkv, n_past)
    return out


# ----------------------------------------------------------------------------
# ops around the path and the whole Qwen3 step (oracle_model.c)
# ----------------------------------------------------------------------------

class _Hparams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in ("n_layer", "n_embd", "n_head", "n_head_kv",
                                              "head_dim", "n_ff", "n_vocab", "n_ctx_train")] + \
               [("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float)]


_LAYER_FIELDS = ("attn_norm", "wq", "wk", "wv", "q_norm", "k_norm", "wo", "ffn_norm", "ffn_gate",
                 "ffn_up", "ffn_down")
# GGUF tensor name suffix of each oracle layer field (src/model.cpp:192-306)
_LAYER_NAMES = {"attn_norm": "attn_norm", "wq": "attn_q", "wk": "attn_k", "wv": "attn_v",
                "q_norm": "attn_q_norm", "k_norm": "attn_k_norm", "wo": "attn_output",
                "ffn_norm": "ffn_norm", "ffn_gate": "ffn_gate", "ffn_up": "ffn_up",
                "ffn_down": "ffn_down"}


class _Layer(ctypes.Structure):
    _fields_ = [(n, _P) for n in _LAYER_FIELDS]


def _model_sigs(lib):
    if getattr(lib, "_model_sigs", False):
        return
    lib.oracle_get_rows_f32.restype = ctypes.c_int
    lib.oracle_get_rows_f32.argtypes = [_P, _P, _P, _I64, _I64, _I64]
    lib.oracle_mul_mat_f32.restype = None
    lib.oracle_mul_mat_f32.argtypes = [_P, _P, _P, _I64, _I64, _I64]
    for n in ("oracle_add_f32", "oracle_mul_f32"):
        getattr(lib, n).restype = None
        getattr(lib, n).argtypes = [_P, _P, _P, _I64]
    lib.oracle_silu_f32.restype = None
    lib.oracle_silu_f32.argtypes = [_P, _P, _I64]
    lib.oracle_sample_greedy.restype = ctypes.c_int32
    lib.oracle_sample_greedy.argtypes = [_P, _I64]
    lib.oracle_qwen3_step.restype = ctypes.c_int
    lib.oracle_qwen3_step.argtypes = [ctypes.POINTER(_Hparams), ctypes.POINTER(_Layer), _P, _P, _P,
                                      _P, _P, _I64, _I64, ctypes.POINTER(_P), ctypes.POINTER(_P),
                                      _P, ctypes.c_int]
    lib._model_sigs = True


def _lib_model():
    lib = load()
    _model_sigs(lib)
    return lib


def get_rows(table, ids):
    table = _f32(table)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty((ids.size, table.shape[1]), dtype=np.float32)
    rc = _lib_model().oracle_get_rows_f32(table.ctypes.data, ids.ctypes.data, out.ctypes.data,
                                          ids.size, table.shape[1], table.shape[0])
    if rc != 0:
        raise ValueError("get_rows: id outside the table")
    return out


def mul_mat(w, x):
    """out[m, n] = sum_k x[m, k] w[n, k] (reference order); x [m, k] or [k]."""
    w = _f32(w)
    x = _f32(x)
    n_out, k = w.shape
    m = x.size // k
    out = np.empty((m, n_out) if x.ndim > 1 else (n_out,), dtype=np.float32)
    _lib_model().oracle_mul_mat_f32(w.ctypes.data, x.ctypes.data, out.ctypes.data, n_out, k, m)
    return out


def elementwise(op, a, b=None):
    a = _f32(a)
    out = np.empty_like(a)
    lib = _lib_model()
    if op == "silu":
        lib.oracle_silu_f32(a.ctypes.data, out.ctypes.data, a.size)
    else:
        b = _f32(b)
        getattr(lib, f"oracle_{op}_f32")(a.ctypes.data, b.ctypes.data, out.ctypes.data, a.size)
    return out


def sample_greedy(logits):
    logits = _f32(logits)
    return int(_lib_model().oracle_sample_greedy(logits.ctypes.data, logits.size))


class Qwen3Oracle:
    """The restated reference CPU backend running a whole Qwen3 model: one
    oracle_qwen3_step per evaluated step, greedy sampling of the last row, the
    generation loop of benchmarks/cpu/bench.cpp:239-281."""

    def __init__(self, cfg, weights, capacity):
        self.cfg = cfg
        self.w = {k: _f32(v) for k, v in weights.items()}
        self.capacity = capacity
        hp = _Hparams(cfg.n_layer, cfg.n_embd, cfg.n_head, cfg.n_head_kv, cfg.head_dim, cfg.n_ff,
                      cfg.n_vocab, cfg.n_ctx_train, cfg.rms_norm_eps, cfg.rope_theta)
        self.hp = hp
        self.layers = (_Layer * cfg.n_layer)()
        for i in range(cfg.n_layer):
            for f in _LAYER_FIELDS:
                setattr(self.layers[i], f, self.w[f"blk.{i}.{_LAYER_NAMES[f]}.weight"].ctypes.data)
        self.theta = rope_theta_table(cfg.rope_theta, cfg.head_dim, cfg.n_ctx_train)
        kv = capacity * cfg.n_head_kv * cfg.head_dim
        self.k = [np.zeros(kv, np.float32) for _ in range(cfg.n_layer)]
        self.v = [np.zeros(kv, np.float32) for _ in range(cfg.n_layer)]
        self.kp = (_P * cfg.n_layer)(*[a.ctypes.data for a in self.k])
        self.vp = (_P * cfg.n_layer)(*[a.ctypes.data for a in self.v])

    def step(self, tokens, n_past, last_row_only=True):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        logits = np.zeros((tokens.size, self.cfg.n_vocab), np.float32)
        emb = self.w["token_embd.weight"]
        # output.weight when the model has one, else the tied embedding
        # (src/model.cpp:203-210)
        out_w = self.w.get("output.weight", emb)
        rc = _lib_model().oracle_qwen3_step(
            ctypes.byref(self.hp), self.layers, emb.ctypes.data,
            self.w["output_norm.weight"].ctypes.data, out_w.ctypes.data, self.theta.ctypes.data,
            tokens.ctypes.data, tokens.size, n_past, self.kp, self.vp, logits.ctypes.data,
            1 if last_row_only else 0)
        if rc != 0:
            raise RuntimeError(f"oracle_qwen3_step returned {rc}")
        return logits

    def generate(self, prompt, n_gen, keep_logits=()):
        """Greedy tokens (benchmarks/cpu/bench.cpp:239-281); the logits row the
        sampler read at each step in keep_logits lands in self.kept[step]."""
        ids = list(prompt)
        n_past = 0
        out = []
        self.kept = {}
        for i in range(n_gen):
            logits = self.step(ids, n_past)
            if i in keep_logits:
                self.kept[i] = logits[-1].copy()
            tok = sample_greedy(logits[-1])
            if tok < 0:
                raise RuntimeError("greedy sampling rejected the logits")
            out.append(tok)
            n_past += len(ids)
            ids = [tok]
        return out
