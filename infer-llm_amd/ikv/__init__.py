"""ikv — Python bindings for the MI355X KV-cache hot path.

Thin ctypes layer over the C-ABI declared in ``include/ikv.h`` and built into
``infer-llm_amd/lib/libikv.so``. PyTorch is used only as plumbing: device
buffers and the current HIP stream. Every call goes to the HIP kernels; there
is no CPU fallback, and loading fails loudly when the library is missing.

Return codes follow ikv.h: 0 ok, negative errno for rejected arguments,
positive hipError_t for a failed launch. Non-zero codes raise ``IkvError``.
"""
from __future__ import annotations

import ctypes
import errno
import os
import pathlib
import re
from typing import Optional

PKG_ROOT = pathlib.Path(__file__).resolve().parents[1]  # infer-llm_amd/
REPO_ROOT = PKG_ROOT.parent
LIB_PATH = PKG_ROOT / "lib" / "libikv.so"
HEADER_DIR = REPO_ROOT / "include"

_c_void_p = ctypes.c_void_p
_c_size_t = ctypes.c_size_t
_c_int = ctypes.c_int
_c_int64 = ctypes.c_int64
_c_float = ctypes.c_float


class KvPages(ctypes.Structure):
    """ikv_kv_pages (include/ikv.h): a paged KV pool's block table."""
    _fields_ = [("block_table", ctypes.c_void_p), ("block_tokens", ctypes.c_int64),
                ("n_pool_blocks", ctypes.c_int64), ("status", ctypes.c_void_p)]


_c_pages = ctypes.POINTER(KvPages)

# name -> (restype, argtypes); include/ikv.h, then include/ikv_model.h
SIGNATURES = {
    "ikv_version": (ctypes.c_char_p, []),
    "ikv_append_f32": (_c_int, [_c_void_p, _c_void_p, _c_size_t, _c_size_t, _c_void_p]),
    "ikv_attn_decode_workspace_bytes": (_c_size_t, [_c_int, _c_int, _c_int, _c_int64]),
    "ikv_attn_decode_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_int, _c_int, _c_int, _c_int64, _c_float, _c_void_p, _c_size_t, _c_void_p],
    ),
    "ikv_attn_decode_noalloc_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_int, _c_int, _c_int, _c_int64, _c_float, _c_void_p],
    ),
    "ikv_attn_decode_rope_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
         _c_int64, _c_float, _c_void_p, _c_void_p, _c_float, _c_void_p, _c_void_p, _c_void_p,
         _c_int64, _c_void_p, _c_void_p, _c_size_t, _c_void_p],
    ),
    "ikv_qkv_attn_decode_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_float, _c_void_p, _c_void_p,
         _c_void_p, _c_int64, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int64,
         _c_float, _c_void_p, _c_void_p, _c_float, _c_void_p, _c_void_p, _c_void_p, _c_int64,
         _c_void_p, _c_void_p, _c_size_t, _c_void_p],
    ),
    "ikv_qkv_attn_decode_replay_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_float, _c_void_p, _c_void_p,
         _c_void_p, _c_int64, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int64,
         _c_float, _c_void_p, _c_void_p, _c_float, _c_void_p, _c_void_p, _c_void_p, _c_int64,
         _c_void_p, _c_void_p, _c_size_t, _c_void_p],
    ),
    "ikv_attn_decode_rope_replay_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
         _c_int64, _c_float, _c_void_p, _c_void_p, _c_float, _c_void_p, _c_void_p, _c_void_p,
         _c_int64, _c_void_p, _c_void_p, _c_size_t, _c_void_p],
    ),
    "ikv_attn_decode_replay_limit": (_c_int64, [_c_int, _c_int, _c_int, _c_int64, _c_int64]),
    "ikv_attn_prefill_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
         _c_int64, _c_int64, _c_int64, _c_float, _c_void_p],
    ),
    "ikv_append_paged_f32": (
        _c_int, [_c_void_p, _c_void_p, _c_pages, _c_int64, _c_size_t, _c_size_t, _c_void_p]),
    "ikv_attn_decode_paged_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_pages, _c_void_p, _c_void_p, _c_void_p,
         _c_int, _c_int, _c_int, _c_int64, _c_float, _c_void_p, _c_size_t, _c_void_p],
    ),
    "ikv_attn_decode_rope_paged_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_pages, _c_void_p, _c_int,
         _c_int, _c_int, _c_int64, _c_float, _c_void_p, _c_void_p, _c_float, _c_void_p,
         _c_void_p, _c_void_p, _c_int64, _c_void_p, _c_void_p, _c_size_t, _c_void_p],
    ),
    "ikv_attn_decode_rope_paged_replay_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_pages, _c_void_p, _c_int,
         _c_int, _c_int, _c_int64, _c_float, _c_void_p, _c_void_p, _c_float, _c_void_p,
         _c_void_p, _c_void_p, _c_int64, _c_void_p, _c_void_p, _c_size_t, _c_void_p],
    ),
    "ikv_attn_prefill_paged_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_pages, _c_void_p, _c_int, _c_int, _c_int,
         _c_int64, _c_int64, _c_int64, _c_float, _c_void_p],
    ),
    "ikv_rms_norm_f32": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int64, _c_int64, _c_float, _c_void_p]),
    "ikv_rope_theta_table_f32": (_c_int, [_c_float, _c_int, _c_int64, _c_void_p]),
    "ikv_rope_sincos_table_f32": (_c_int, [_c_void_p, _c_size_t, _c_void_p, _c_void_p]),
    "ikv_rope_neox_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_int64, _c_int, _c_int, _c_void_p, _c_void_p,
         _c_int64, _c_void_p, _c_void_p],
    ),
    "ikv_qk_norm_rope_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int64, _c_int, _c_int, _c_float,
         _c_void_p, _c_void_p, _c_int64, _c_void_p, _c_void_p],
    ),
    # include/ikv_model.h
    "ikv_mul_mat_f32": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int64, _c_int64, _c_int64, _c_void_p, _c_void_p]),
    "ikv_gemm_nt_f32": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int64, _c_int64, _c_int64, _c_void_p, _c_void_p]),
    "ikv_gemv3_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_int64, _c_int64, _c_int64, _c_int64, _c_void_p, _c_float, _c_void_p],
    ),
    "ikv_gemv_swiglu_f32": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int64, _c_int64, _c_void_p, _c_float,
                 _c_void_p]),
    "ikv_get_rows_f32": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_int64, _c_int64, _c_int64, _c_void_p, _c_void_p]),
    "ikv_add_f32": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int64, _c_void_p]),
    "ikv_mul_f32": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int64, _c_void_p]),
    "ikv_silu_f32": (_c_int, [_c_void_p, _c_void_p, _c_int64, _c_void_p]),
    "ikv_silu_mul_f32": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int64, _c_void_p]),
    "ikv_argmax_f32": (_c_int, [_c_void_p, _c_int64, _c_void_p, _c_void_p, _c_void_p]),
    "ikv_argmax_workspace_bytes": (_c_size_t, []),
    "ikv_argmax_ws_f32": (
        _c_int, [_c_void_p, _c_int64, _c_void_p, _c_void_p, _c_void_p, _c_size_t, _c_void_p]),
    "ikv_synth_normal_f32": (
        _c_int, [ctypes.c_uint64, ctypes.c_uint64, _c_size_t, ctypes.c_double, _c_void_p, _c_int]),
}

# libikv_bench.so, the measurement library (infer-llm_amd/bench/ikv_bench.h):
# its own entry points; its decode build also has include/ikv.h's decode ones
BENCH_LIB_PATH = PKG_ROOT / "lib" / "libikv_bench.so"
BENCH_HEADER = PKG_ROOT / "bench" / "ikv_bench.h"
BENCH_SIGNATURES = {
    "ikv_probe_read": (_c_int, [_c_void_p, _c_size_t, _c_void_p, _c_int, _c_int, _c_void_p]),
    "ikv_probe_empty": (_c_int, [_c_int, _c_void_p]),
    "ikv_bench_timeline_read": (_c_int, [_c_void_p, _c_size_t]),
    "ikv_bench_timeline_clear": (_c_int, []),
    "ikv_bench_gemm_nt_tile_f32": (
        _c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int64, _c_int64, _c_int64, _c_void_p, _c_int,
                 _c_int, _c_void_p, _c_size_t, _c_void_p]),
    "ikv_bench_gemm_plan": (_c_int, [_c_int64, _c_int64, _c_int64, _c_void_p, _c_void_p]),
}


class IkvError(RuntimeError):
    """A C-ABI entry point returned a non-zero code."""

    def __init__(self, fn: str, rc: int):
        self.fn, self.rc = fn, rc
        if rc < 0:
            what = errno.errorcode.get(-rc, str(-rc))
            super().__init__(f"{fn} rejected its arguments: -{what}")
        else:
            super().__init__(f"{fn} launch failed: hipError_t {rc}")


_lib: Optional[ctypes.CDLL] = None
_bench_lib: Optional[ctypes.CDLL] = None


def header_functions() -> list[str]:
    """Names of the entry points declared in include/*.h."""
    names = set()
    for h in sorted(HEADER_DIR.glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(ikv_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def load_bench() -> ctypes.CDLL:
    """Load libikv_bench.so (once): the probes, the timeline reader, and the
    stamped decode build's entry points (with include/ikv.h's signatures).
    Its own symbols stay local to its handle, apart from libikv.so's."""
    global _bench_lib
    if _bench_lib is not None:
        return _bench_lib
    if not BENCH_LIB_PATH.exists():
        raise FileNotFoundError(f"{BENCH_LIB_PATH} is not built")
    lib = ctypes.CDLL(str(BENCH_LIB_PATH))
    for name, (res, args) in BENCH_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    for name in ("ikv_attn_decode_f32", "ikv_attn_decode_workspace_bytes"):
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = SIGNATURES[name]
    _bench_lib = lib
    return lib


def load() -> ctypes.CDLL:
    """Load libikv.so (once). Raises if the library has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise FileNotFoundError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _check(fn: str, rc: int) -> None:
    if rc != 0:
        raise IkvError(fn, rc)


# ----------------------------------------------------------------------------
# torch plumbing
# ----------------------------------------------------------------------------

def _torch():
    import torch  # imported lazily so CPU-only users of the ABI need no torch
    return torch


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(stream=None) -> int:
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def _need_f32_dev(name: str, t) -> None:
    torch = _torch()
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


# ----------------------------------------------------------------------------
# entry points
# ----------------------------------------------------------------------------

def version() -> str:
    return load().ikv_version().decode()


def append(dst_rows, src_rows, stream=None) -> None:
    """KV append: copy src_rows into dst_rows (both contiguous device tensors of
    equal byte size; dst_rows is the writable cache view)."""
    _need_f32_dev("dst_rows", dst_rows)
    _need_f32_dev("src_rows", src_rows)
    if dst_rows.numel() != src_rows.numel():
        raise ValueError("append: size mismatch")
    n_rows = src_rows.shape[0] if src_rows.dim() > 0 else 1
    row_bytes = src_rows.numel() * 4 // max(n_rows, 1)
    _check("ikv_append_f32",
           load().ikv_append_f32(_ptr(dst_rows), _ptr(src_rows), n_rows, row_bytes, _stream(stream)))


def decode_replay_limit(n_head: int, n_head_kv: int, head_dim: int, n_kv: int, width: int) -> int:
    return int(load().ikv_attn_decode_replay_limit(n_head, n_head_kv, head_dim, n_kv, width))


def decode_workspace_bytes(n_head: int, n_head_kv: int, head_dim: int, n_kv: int) -> int:
    return int(load().ikv_attn_decode_workspace_bytes(n_head, n_head_kv, head_dim, n_kv))


def decode_workspace(n_head: int, n_head_kv: int, head_dim: int, n_kv: int, device="cuda"):
    """Zero-filled workspace for attn_decode at every context up to n_kv
    (reusable across ordered launches). The split count is not monotone in
    the context (it peaks where a split's tile count steps down), so every
    context is asked."""
    torch = _torch()
    nbytes = 256
    for n in range(1, n_kv + 1):
        nbytes = max(nbytes, decode_workspace_bytes(n_head, n_head_kv, head_dim, n))
    return torch.zeros((nbytes + 3) // 4, dtype=torch.float32, device=device)


def attn_decode(q, k_cache, v_cache, n_kv: int, *, k_new=None, v_new=None, out=None,
                scale: float = 0.0, workspace=None, stream=None):
    """Decode attention for one query token over cache rows [0, n_kv).

    q: [n_head, D]; k_cache/v_cache: [capacity, n_head_kv, D]; when k_new/v_new
    ([n_head_kv, D]) are given, row n_kv-1 is taken from them and appended."""
    torch = _torch()
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        _need_f32_dev(name, t)
    n_head, D = q.shape[-2], q.shape[-1]
    n_head_kv = k_cache.shape[-2]
    if k_cache.shape[0] < n_kv or v_cache.shape[0] < n_kv:
        raise ValueError("cache shorter than n_kv")
    if (k_new is None) != (v_new is None):
        raise ValueError("k_new and v_new go together")
    if k_new is not None:
        _need_f32_dev("k_new", k_new)
        _need_f32_dev("v_new", v_new)
        if k_new.numel() != n_head_kv * D or v_new.numel() != n_head_kv * D:
            raise ValueError("k_new/v_new must hold one token row")
    if out is None:
        out = torch.empty((n_head, D), dtype=torch.float32, device=q.device)
    _need_f32_dev("out", out)
    if workspace is None:
        workspace = decode_workspace(n_head, n_head_kv, D, n_kv, device=q.device)
    rc = load().ikv_attn_decode_f32(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(k_new), _ptr(v_new), _ptr(out),
        n_head, n_head_kv, D, n_kv, scale, _ptr(workspace), workspace.numel() * 4, _stream(stream))
    _check("ikv_attn_decode_f32", rc)
    return out


# IKV_STATUS_* bits (include/ikv.h) a kernel raises in a device status word
STATUS_POSITION, STATUS_BLOCK, STATUS_TOKEN = 1, 2, 4

# IKV_DECODE_NOALLOC_SCRATCH_BYTES (include/ikv.h): the device array that
# attn_decode_noalloc keeps its split partials and counters in
NOALLOC_SCRATCH_BYTES = 2 << 20


def attn_decode_noalloc(q, k_cache, v_cache, n_kv: int, *, out, k_new=None, v_new=None,
                        scale: float = 0.0, stream=None):
    """attn_decode without a workspace: nothing is allocated (out is the
    caller's). The library's per-device scratch array holds the split
    partials, so calls on one device must be ordered on one stream."""
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache), ("out", out)):
        _need_f32_dev(name, t)
    n_head, D = q.shape[-2], q.shape[-1]
    n_head_kv = k_cache.shape[-2]
    if k_cache.shape[0] < n_kv or v_cache.shape[0] < n_kv:
        raise ValueError("cache shorter than n_kv")
    if (k_new is None) != (v_new is None):
        raise ValueError("k_new and v_new go together")
    if k_new is not None:
        _need_f32_dev("k_new", k_new)
        _need_f32_dev("v_new", v_new)
        if k_new.numel() != n_head_kv * D or v_new.numel() != n_head_kv * D:
            raise ValueError("k_new/v_new must hold one token row")
    if out.numel() != n_head * D:
        raise ValueError("out must hold n_head rows")
    rc = load().ikv_attn_decode_noalloc_f32(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(k_new), _ptr(v_new), _ptr(out),
        n_head, n_head_kv, D, n_kv, scale, _stream(stream))
    _check("ikv_attn_decode_noalloc_f32", rc)
    return out


def qkv_attn_decode(w_q, w_k, w_v, x, k_cache, v_cache, n_kv: int, q_norm_w, k_norm_w,
                    eps: float, pos, sin_tab, cos_tab, *, attn_norm_w=None, attn_eps: float = 0.0,
                    q_out=None, k_out=None, v_out=None, out=None, scale: float = 0.0, status=None,
                    workspace=None, replay=False, stream=None):
    """One token's q/k/v projections (attn_norm folded in when attn_norm_w is
    given) and its decode (qk-norm + RoPE + append + attention) in one launch,
    for contexts of one decode split. Returns (out, q_out, k_out, v_out).
    replay=True: the replay form, n_kv is then the planned maximum and the
    context is pos[0] + 1, read on the device."""
    torch = _torch()
    n_embd = x.numel()
    D = k_cache.shape[-1]
    n_head_kv = k_cache.shape[-2]
    n_head = w_q.shape[0] // D
    dev = x.device
    if q_out is None:
        q_out = torch.empty((n_head, D), dtype=torch.float32, device=dev)
    if k_out is None:
        k_out = torch.empty((n_head_kv, D), dtype=torch.float32, device=dev)
    if v_out is None:
        v_out = torch.empty((n_head_kv, D), dtype=torch.float32, device=dev)
    if out is None:
        out = torch.empty((n_head, D), dtype=torch.float32, device=dev)
    if workspace is None:
        workspace = decode_workspace(n_head, n_head_kv, D, n_kv, device=dev)
    fn = "ikv_qkv_attn_decode_replay_f32" if replay else "ikv_qkv_attn_decode_f32"
    rc = getattr(load(), fn)(
        _ptr(w_q), _ptr(w_k), _ptr(w_v), _ptr(x), _ptr(attn_norm_w), attn_eps, _ptr(q_out),
        _ptr(k_out), _ptr(v_out), n_embd, _ptr(k_cache), _ptr(v_cache), _ptr(out), n_head,
        n_head_kv, D, n_kv, scale, _ptr(q_norm_w), _ptr(k_norm_w), eps, _ptr(pos), _ptr(sin_tab),
        _ptr(cos_tab), sin_tab.shape[0], _ptr(status), _ptr(workspace), workspace.numel() * 4,
        _stream(stream))
    _check(fn, rc)
    return out, q_out, k_out, v_out


def attn_decode_rope(q_raw, k_raw, v_new, k_cache, v_cache, n_kv: int, q_norm_w, k_norm_w,
                     eps: float, pos, sin_tab, cos_tab, *, out=None, scale: float = 0.0,
                     status=None, workspace=None, replay=False, stream=None):
    """Decode with qk-RMSNorm + RoPE folded in: q/k rotated at position pos[0],
    k (rotated) and v_new appended at row n_kv-1, attention over [0, n_kv).
    replay=True: the replay form, n_kv is then the planned maximum and the
    context is pos[0] + 1, read on the device."""
    torch = _torch()
    n_head, D = q_raw.shape[-2], q_raw.shape[-1]
    n_head_kv = k_cache.shape[-2]
    if out is None:
        out = torch.empty((n_head, D), dtype=torch.float32, device=q_raw.device)
    if workspace is None:
        workspace = decode_workspace(n_head, n_head_kv, D, n_kv, device=q_raw.device)
    fn = "ikv_attn_decode_rope_replay_f32" if replay else "ikv_attn_decode_rope_f32"
    rc = getattr(load(), fn)(
        _ptr(q_raw), _ptr(k_raw), _ptr(v_new), _ptr(k_cache), _ptr(v_cache), _ptr(out), n_head,
        n_head_kv, D, n_kv, scale, _ptr(q_norm_w), _ptr(k_norm_w), eps, _ptr(pos), _ptr(sin_tab),
        _ptr(cos_tab), sin_tab.shape[0], _ptr(status), _ptr(workspace), workspace.numel() * 4,
        _stream(stream))
    _check(fn, rc)
    return out


def attn_prefill(q, k, v, n_past: int = 0, *, n_kv: Optional[int] = None, out=None,
                 scale: float = 0.0, stream=None):
    """Causal attention for q [n_q, n_head, D] over k, v [>= n_kv, n_head_kv, D]."""
    torch = _torch()
    for name, t in (("q", q), ("k", k), ("v", v)):
        _need_f32_dev(name, t)
    n_q, n_head, D = q.shape
    n_head_kv = k.shape[1]
    if n_kv is None:
        n_kv = n_past + n_q
    if out is None:
        out = torch.empty_like(q)
    _need_f32_dev("out", out)
    rc = load().ikv_attn_prefill_f32(_ptr(q), _ptr(k), _ptr(v), _ptr(out), n_head, n_head_kv, D,
                                     n_q, n_kv, n_past, scale, _stream(stream))
    _check("ikv_attn_prefill_f32", rc)
    return out


# ----------------------------------------------------------------------------
# paged KV pool: [n_blocks * block_tokens, n_head_kv, D] per K and V; logical
# token t in pool row table[t // block_tokens] * block_tokens + t % block_tokens
# ----------------------------------------------------------------------------

def kv_pages(table, block_tokens: int, pool, status=None) -> KvPages:
    """The ikv_kv_pages descriptor of a device int32 block table over `pool`."""
    torch = _torch()
    if table.dtype != torch.int32 or not table.is_cuda or not table.is_contiguous():
        raise ValueError("block table must be a contiguous device int32 tensor")
    if pool.shape[0] % block_tokens:
        raise ValueError("pool rows must be whole blocks")
    return KvPages(table.data_ptr(), block_tokens, pool.shape[0] // block_tokens, _ptr(status))


def append_paged(pool, src_rows, table, block_tokens: int, first_token: int, status=None,
                 stream=None) -> None:
    """Writes src_rows [n, n_head_kv, D] to logical tokens first_token.. of the pool."""
    _need_f32_dev("pool", pool)
    _need_f32_dev("src_rows", src_rows)
    n_rows = src_rows.shape[0]
    row_bytes = src_rows[0].numel() * 4 if n_rows else 0
    pg = kv_pages(table, block_tokens, pool, status)
    _check("ikv_append_paged_f32",
           load().ikv_append_paged_f32(_ptr(pool), _ptr(src_rows), ctypes.byref(pg), first_token,
                                       n_rows, row_bytes, _stream(stream)))


def attn_decode_paged(q, k_pool, v_pool, table, block_tokens: int, n_kv: int, *, k_new=None,
                      v_new=None, out=None, scale: float = 0.0, status=None, workspace=None,
                      stream=None):
    """attn_decode over a paged pool (logical rows [0, n_kv) through `table`)."""
    torch = _torch()
    for name, t in (("q", q), ("k_pool", k_pool), ("v_pool", v_pool)):
        _need_f32_dev(name, t)
    n_head, D = q.shape[-2], q.shape[-1]
    n_head_kv = k_pool.shape[-2]
    if out is None:
        out = torch.empty((n_head, D), dtype=torch.float32, device=q.device)
    if workspace is None:
        workspace = decode_workspace(n_head, n_head_kv, D, n_kv, device=q.device)
    pg = kv_pages(table, block_tokens, k_pool, status)
    rc = load().ikv_attn_decode_paged_f32(
        _ptr(q), _ptr(k_pool), _ptr(v_pool), ctypes.byref(pg), _ptr(k_new), _ptr(v_new),
        _ptr(out), n_head, n_head_kv, D, n_kv, scale, _ptr(workspace), workspace.numel() * 4,
        _stream(stream))
    _check("ikv_attn_decode_paged_f32", rc)
    return out


def attn_decode_rope_paged(q_raw, k_raw, v_new, k_pool, v_pool, table, block_tokens: int,
                           n_kv: int, q_norm_w, k_norm_w, eps: float, pos, sin_tab, cos_tab, *,
                           out=None, scale: float = 0.0, status=None, page_status=None,
                           workspace=None, replay=False, stream=None):
    """attn_decode_rope over a paged pool (replay=True: the replay form, n_kv
    the planned maximum, the context pos[0] + 1 read on the device)."""
    torch = _torch()
    n_head, D = q_raw.shape[-2], q_raw.shape[-1]
    n_head_kv = k_pool.shape[-2]
    if out is None:
        out = torch.empty((n_head, D), dtype=torch.float32, device=q_raw.device)
    if workspace is None:
        workspace = decode_workspace(n_head, n_head_kv, D, n_kv, device=q_raw.device)
    pg = kv_pages(table, block_tokens, k_pool, page_status)
    fn = "ikv_attn_decode_rope_paged_replay_f32" if replay else "ikv_attn_decode_rope_paged_f32"
    rc = getattr(load(), fn)(
        _ptr(q_raw), _ptr(k_raw), _ptr(v_new), _ptr(k_pool), _ptr(v_pool), ctypes.byref(pg),
        _ptr(out), n_head, n_head_kv, D, n_kv, scale, _ptr(q_norm_w), _ptr(k_norm_w), eps,
        _ptr(pos), _ptr(sin_tab), _ptr(cos_tab), sin_tab.shape[0], _ptr(status), _ptr(workspace),
        workspace.numel() * 4, _stream(stream))
    _check(fn, rc)
    return out


def attn_prefill_paged(q, k_pool, v_pool, table, block_tokens: int, n_past: int = 0, *,
                       n_kv: Optional[int] = None, out=None, scale: float = 0.0, status=None,
                       stream=None):
    """attn_prefill over a paged pool."""
    torch = _torch()
    for name, t in (("q", q), ("k_pool", k_pool), ("v_pool", v_pool)):
        _need_f32_dev(name, t)
    n_q, n_head, D = q.shape
    n_head_kv = k_pool.shape[1]
    if n_kv is None:
        n_kv = n_past + n_q
    if out is None:
        out = torch.empty_like(q)
    pg = kv_pages(table, block_tokens, k_pool, status)
    rc = load().ikv_attn_prefill_paged_f32(_ptr(q), _ptr(k_pool), _ptr(v_pool), ctypes.byref(pg),
                                           _ptr(out), n_head, n_head_kv, D, n_q, n_kv, n_past,
                                           scale, _stream(stream))
    _check("ikv_attn_prefill_paged_f32", rc)
    return out


def rms_norm(x, w, eps: float, out=None, stream=None):
    torch = _torch()
    _need_f32_dev("x", x)
    _need_f32_dev("w", w)
    dim = x.shape[-1]
    if w.numel() != dim:
        raise ValueError("weight length must equal the last dim")
    if out is None:
        out = torch.empty_like(x)
    rows = x.numel() // dim
    _check("ikv_rms_norm_f32",
           load().ikv_rms_norm_f32(_ptr(x), _ptr(w), _ptr(out), rows, dim, eps, _stream(stream)))
    return out


def rope_theta_table(theta_base: float, head_dim: int, n_ctx: int):
    """Host RoPE angle table [n_ctx][head_dim/2] (numpy float32), the
    engine's own (GraphContext::get_rope_theta_table)."""
    import numpy as np
    out = np.empty((n_ctx, head_dim // 2), dtype=np.float32)
    _check("ikv_rope_theta_table_f32",
           load().ikv_rope_theta_table_f32(theta_base, head_dim, n_ctx, out.ctypes.data))
    return out


def rope_sincos_table(theta):
    """Host sin/cos tables (numpy float32) from a host angle table."""
    import numpy as np
    theta = np.ascontiguousarray(theta, dtype=np.float32)
    s = np.empty_like(theta)
    c = np.empty_like(theta)
    _check("ikv_rope_sincos_table_f32",
           load().ikv_rope_sincos_table_f32(theta.ctypes.data, theta.size, s.ctypes.data,
                                            c.ctypes.data))
    return s, c


def rope_neox(x, pos, sin_tab, cos_tab, out=None, status=None, stream=None):
    """x: [n_tokens, n_heads, D]; pos: int32 [n_tokens]; tables [n_ctx, D/2]."""
    torch = _torch()
    _need_f32_dev("x", x)
    n_tokens, n_heads, D = x.shape
    if out is None:
        out = torch.empty_like(x)
    rc = load().ikv_rope_neox_f32(_ptr(x), _ptr(out), _ptr(pos), n_tokens, n_heads, D,
                                  _ptr(sin_tab), _ptr(cos_tab), sin_tab.shape[0], _ptr(status),
                                  _stream(stream))
    _check("ikv_rope_neox_f32", rc)
    return out


def qk_norm_rope(x, w, pos, eps: float, sin_tab, cos_tab, out=None, status=None, stream=None):
    torch = _torch()
    _need_f32_dev("x", x)
    n_tokens, n_heads, D = x.shape
    if out is None:
        out = torch.empty_like(x)
    rc = load().ikv_qk_norm_rope_f32(_ptr(x), _ptr(w), _ptr(out), _ptr(pos), n_tokens, n_heads, D,
                                     eps, _ptr(sin_tab), _ptr(cos_tab), sin_tab.shape[0],
                                     _ptr(status), _stream(stream))
    _check("ikv_qk_norm_rope_f32", rc)
    return out


# ----------------------------------------------------------------------------
# ops around the path (include/ikv_model.h)
# ----------------------------------------------------------------------------

def mul_mat(w, x, out=None, residual=None, stream=None):
    """out[m, n] = x[m, :] . w[n, :] (+ residual); w [n_out, k], x [m, k] or [k]."""
    torch = _torch()
    _need_f32_dev("w", w)
    _need_f32_dev("x", x)
    n_out, k = w.shape
    m = x.numel() // k
    if x.numel() != m * k:
        raise ValueError("x length must be a multiple of k")
    if out is None:
        out = torch.empty((m, n_out) if x.dim() > 1 else (n_out,), device=x.device)
    _check("ikv_mul_mat_f32", load().ikv_mul_mat_f32(_ptr(w), _ptr(x), _ptr(out), n_out, k, m,
                                                      _ptr(residual), _stream(stream)))
    return out


def gemm_nt(w, x, out=None, residual=None, stream=None):
    """The MFMA GEMM of mul_mat for any number of tokens: out[m, n] =
    x[m, :] . w[n, :] (+ residual); n_out % 64 == 0 and k % 64 == 0."""
    torch = _torch()
    _need_f32_dev("w", w)
    _need_f32_dev("x", x)
    n_out, k = w.shape
    m = x.numel() // k
    if x.numel() != m * k:
        raise ValueError("x length must be a multiple of k")
    if out is None:
        out = torch.empty((m, n_out), device=x.device)
    _check("ikv_gemm_nt_f32", load().ikv_gemm_nt_f32(_ptr(w), _ptr(x), _ptr(out), n_out, k, m,
                                                      _ptr(residual), _stream(stream)))
    return out


def gemv3(w0, w1, w2, x, norm_w=None, eps: float = 1e-6, stream=None):
    """[w_i . x'] for i = 0, 1, 2; x' = rms_norm(x, norm_w, eps) when norm_w is given."""
    torch = _torch()
    k = x.numel()
    outs = [torch.empty(w.shape[0], device=x.device) for w in (w0, w1, w2)]
    _check("ikv_gemv3_f32", load().ikv_gemv3_f32(
        _ptr(w0), _ptr(w1), _ptr(w2), _ptr(x), _ptr(outs[0]), _ptr(outs[1]), _ptr(outs[2]),
        w0.shape[0], w1.shape[0], w2.shape[0], k, _ptr(norm_w), eps, _stream(stream)))
    return outs


def gemv_swiglu(w_gate, w_up, x, out=None, norm_w=None, eps: float = 1e-6, stream=None):
    torch = _torch()
    n_out, k = w_gate.shape
    if out is None:
        out = torch.empty(n_out, device=x.device)
    _check("ikv_gemv_swiglu_f32", load().ikv_gemv_swiglu_f32(
        _ptr(w_gate), _ptr(w_up), _ptr(x), _ptr(out), n_out, k, _ptr(norm_w), eps,
        _stream(stream)))
    return out


def get_rows(table, ids, out=None, status=None, stream=None):
    torch = _torch()
    n_rows, row_len = table.shape
    if out is None:
        out = torch.empty((ids.numel(), row_len), device=table.device)
    _check("ikv_get_rows_f32", load().ikv_get_rows_f32(
        _ptr(table), _ptr(ids), _ptr(out), ids.numel(), row_len, n_rows, _ptr(status),
        _stream(stream)))
    return out


def elementwise(op: str, a, b=None, out=None, stream=None):
    torch = _torch()
    if out is None:
        out = torch.empty_like(a)
    lib = load()
    if op == "silu":
        rc = lib.ikv_silu_f32(_ptr(a), _ptr(out), a.numel(), _stream(stream))
    else:
        rc = getattr(lib, f"ikv_{op}_f32")(_ptr(a), _ptr(b), _ptr(out), a.numel(), _stream(stream))
    _check(f"ikv_{op}_f32", rc)
    return out


def argmax(logits, token=None, mirror=None, workspace=None, stream=None):
    """Device int32 [1]: greedy token of logits (ties -> lowest id; -1 on NaN/+inf);
    `mirror` (e.g. a pinned host tensor) receives a copy. With `workspace`
    (argmax_workspace()), the multi-workgroup form runs."""
    torch = _torch()
    if token is None:
        token = torch.empty(1, dtype=torch.int32, device=logits.device)
    if workspace is None:
        _check("ikv_argmax_f32", load().ikv_argmax_f32(_ptr(logits), logits.numel(), _ptr(token),
                                                        _ptr(mirror), _stream(stream)))
    else:
        _check("ikv_argmax_ws_f32",
               load().ikv_argmax_ws_f32(_ptr(logits), logits.numel(), _ptr(token), _ptr(mirror),
                                        _ptr(workspace), workspace.numel() * workspace.element_size(),
                                        _stream(stream)))
    return token


def argmax_workspace(device=None):
    """Zeroed device workspace of the multi-workgroup greedy sampler."""
    torch = _torch()
    n = int(load().ikv_argmax_workspace_bytes())
    return torch.zeros(n, dtype=torch.uint8, device=device or "cuda")


def synth_normal(seed: int, shape, std: float = 1.0, offset: int = 0, threads: int = 8):
    """Host float32 N(0, std^2) array from the product's synthetic initialiser."""
    import numpy as np
    out = np.empty(shape, dtype=np.float32)
    _check("ikv_synth_normal_f32", load().ikv_synth_normal_f32(
        seed & 0xFFFFFFFFFFFFFFFF, offset, out.size, std, out.ctypes.data, threads))
    return out
