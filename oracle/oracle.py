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
