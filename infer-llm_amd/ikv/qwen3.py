"""Qwen3 on the HIP backend from Python: the engine's C-ABI (include/ikv_engine.h)
and the benchmark configurations' synthetic weights.

Qwen3Engine wraps ikv_qwen3_*: a Qwen3Model graph (src/models/Qwen3.cpp:4-136)
executed by the engine's Scheduler on HIPBackend with the KV cache in HBM, and
the benchmark runner's greedy loop (benchmarks/cpu/bench.cpp:239-281).
"""
from __future__ import annotations

import ctypes
import dataclasses

import numpy as np

from . import _check, load


@dataclasses.dataclass(frozen=True)
class Qwen3Config:
    n_layer: int = 28
    n_embd: int = 1024
    n_head: int = 16
    n_head_kv: int = 8
    head_dim: int = 128
    n_ff: int = 3072
    n_vocab: int = 151936
    n_ctx_train: int = 40960
    rope_theta: float = 1e6
    rms_norm_eps: float = 1e-6
    untied_output: int = 0  # 1: a separate output.weight projects the logits


QWEN3_0_6B = Qwen3Config()
QWEN3_8B = Qwen3Config(n_layer=36, n_embd=4096, n_head=32, n_head_kv=8, n_ff=12288)


class _Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("n_layer", "n_embd", "n_head", "n_head_kv",
                                               "head_dim", "n_ff", "n_vocab", "n_ctx_train")] + \
               [("rope_theta", ctypes.c_float), ("rms_norm_eps", ctypes.c_float),
                ("untied_output", ctypes.c_uint32)]


class Timing(ctypes.Structure):
    _fields_ = [(n, ctypes.c_double) for n in ("ttft_s", "tpot_s", "wall_s", "build_s",
                                               "execute_s", "sample_s")]


class Stats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("launches", "fused_norm_rope", "fused_append_decode",
                                            "fused_swiglu", "fused_residual", "fused_qkv",
                                            "fused_norm_mm", "fused_rope_decode",
                                            "fused_qkv_decode", "fused_append",
                                            "step_captures", "step_replays")]


_P = ctypes.c_void_p
class KvStats(ctypes.Structure):
    _fields_ = [(f, ctypes.c_uint64) for f in ("page_ins", "page_outs", "evictions", "bytes_in",
                                                "bytes_out")]


ENGINE_SIGNATURES = {
    "ikv_qwen3_create": (ctypes.c_int, [ctypes.POINTER(_Config), ctypes.c_int, ctypes.c_int64,
                                        ctypes.POINTER(_P)]),
    "ikv_qwen3_create_paged": (ctypes.c_int, [ctypes.POINTER(_Config), ctypes.c_int, ctypes.c_int64,
                                              ctypes.c_int64, ctypes.c_int64, ctypes.POINTER(_P)]),
    "ikv_qwen3_create_offload": (ctypes.c_int, [ctypes.POINTER(_Config), ctypes.c_int, ctypes.c_int64,
                                                ctypes.c_uint64, ctypes.POINTER(_P)]),
    "ikv_qwen3_kv_stats": (ctypes.c_int, [_P, ctypes.POINTER(KvStats)]),
    "ikv_qwen3_tensor_count": (ctypes.c_int, [_P]),
    "ikv_qwen3_tensor_name": (ctypes.c_char_p, [_P, ctypes.c_int]),
    "ikv_qwen3_tensor_size": (ctypes.c_size_t, [_P, ctypes.c_char_p]),
    "ikv_qwen3_set_tensor": (ctypes.c_int, [_P, ctypes.c_char_p, _P, ctypes.c_size_t]),
    "ikv_qwen3_init_synthetic": (ctypes.c_int, [_P, ctypes.c_uint64, ctypes.c_double, ctypes.c_int]),
    "ikv_qwen3_generate": (ctypes.c_int, [_P, _P, ctypes.c_int64, ctypes.c_int64, _P,
                                          ctypes.POINTER(Timing)]),
    "ikv_qwen3_generate_interleaved": (ctypes.c_int, [_P, _P, ctypes.c_int64, ctypes.c_int64,
                                                      ctypes.c_int64, _P, ctypes.POINTER(Timing)]),
    "ikv_qwen3_last_stats": (ctypes.c_int, [_P, ctypes.POINTER(Stats)]),
    "ikv_qwen3_set_fusion": (ctypes.c_int, [_P, ctypes.c_int]),
    "ikv_qwen3_set_step_replay": (ctypes.c_int, [_P, ctypes.c_int]),
    "ikv_qwen3_capture_logits": (ctypes.c_int, [_P, _P, ctypes.c_int64]),
    "ikv_qwen3_captured_logits": (ctypes.c_int, [_P, _P, ctypes.c_size_t]),
    "ikv_qwen3_destroy": (None, [_P]),
}


def _lib():
    lib = load()
    if not getattr(lib, "_engine_sigs", False):
        for name, (res, args) in ENGINE_SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        lib._engine_sigs = True
    return lib


def tensor_layout(cfg: Qwen3Config):
    """(name, shape) of every weight in the engine's order (rows x columns as
    stored: [n_out][n_in] for matrices)."""
    E, D, F = cfg.n_embd, cfg.head_dim, cfg.n_ff
    Q, KV = cfg.n_head * D, cfg.n_head_kv * D
    out = [("token_embd.weight", (cfg.n_vocab, E))]
    for i in range(cfg.n_layer):
        p = f"blk.{i}."
        out += [(p + "attn_norm.weight", (E,)), (p + "attn_q.weight", (Q, E)),
                (p + "attn_k.weight", (KV, E)), (p + "attn_v.weight", (KV, E)),
                (p + "attn_q_norm.weight", (D,)), (p + "attn_k_norm.weight", (D,)),
                (p + "attn_output.weight", (E, Q)), (p + "ffn_norm.weight", (E,)),
                (p + "ffn_gate.weight", (F, E)), (p + "ffn_up.weight", (F, E)),
                (p + "ffn_down.weight", (E, F))]
    out.append(("output_norm.weight", (E,)))
    if cfg.untied_output:
        out.append(("output.weight", (cfg.n_vocab, E)))
    return out


def synthetic_weights(cfg: Qwen3Config, seed: int, std: float = 0.02, threads: int = 8):
    """Host copies of the weights ikv_qwen3_init_synthetic creates: matrices
    N(0, std^2) from one stream in tensor order, norm weights 1.0."""
    from . import synth_normal
    w, offset = {}, 0
    for name, shape in tensor_layout(cfg):
        if "norm" in name:
            w[name] = np.ones(shape, np.float32)
        else:
            w[name] = synth_normal(seed, shape, std, offset=offset, threads=threads)
            offset += int(np.prod(shape))
    return w


class Qwen3Engine:
    """A Qwen3 model on HIP device `device` with a KV cache of max_ctx tokens:
    one contiguous cache per layer; with block_tokens > 0 a paged cache
    (pool_blocks blocks of block_tokens tokens per layer; 0 = max_ctx worth);
    with offload_hbm_bytes > 0 per-layer caches in pinned host memory of which
    at most that many bytes are resident in HBM."""

    def __init__(self, cfg: Qwen3Config, max_ctx: int, device: int = 0, block_tokens: int = 0,
                 pool_blocks: int = 0, offload_hbm_bytes: int = 0):
        self.cfg = cfg
        c = _Config(*(getattr(cfg, f) for f, _ in _Config._fields_))
        h = _P()
        if offload_hbm_bytes:
            _check("ikv_qwen3_create_offload",
                   _lib().ikv_qwen3_create_offload(ctypes.byref(c), device, max_ctx,
                                                   offload_hbm_bytes, ctypes.byref(h)))
        elif block_tokens:
            _check("ikv_qwen3_create_paged",
                   _lib().ikv_qwen3_create_paged(ctypes.byref(c), device, max_ctx, block_tokens,
                                                 pool_blocks, ctypes.byref(h)))
        else:
            _check("ikv_qwen3_create", _lib().ikv_qwen3_create(ctypes.byref(c), device, max_ctx,
                                                               ctypes.byref(h)))
        self._h = h
        self._logit_steps = []

    def close(self):
        if self._h:
            _lib().ikv_qwen3_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def kv_stats(self):
        st = KvStats()
        _check("ikv_qwen3_kv_stats", _lib().ikv_qwen3_kv_stats(self._h, ctypes.byref(st)))
        return {f: getattr(st, f) for f, _ in KvStats._fields_}

    def tensor_names(self):
        lib = _lib()
        return [lib.ikv_qwen3_tensor_name(self._h, i).decode()
                for i in range(lib.ikv_qwen3_tensor_count(self._h))]

    def set_weights(self, weights):
        lib = _lib()
        for name, arr in weights.items():
            arr = np.ascontiguousarray(arr, dtype=np.float32)
            _check("ikv_qwen3_set_tensor", lib.ikv_qwen3_set_tensor(
                self._h, name.encode(), arr.ctypes.data, arr.size))

    def init_synthetic(self, seed: int, std: float = 0.02, threads: int = 8):
        _check("ikv_qwen3_init_synthetic", _lib().ikv_qwen3_init_synthetic(
            self._h, seed & 0xFFFFFFFFFFFFFFFF, std, threads))

    def set_fusion(self, on: bool):
        _check("ikv_qwen3_set_fusion", _lib().ikv_qwen3_set_fusion(self._h, 1 if on else 0))

    def set_step_replay(self, on: bool):
        """Decode steps replayed from a captured HIP graph (default on)."""
        _check("ikv_qwen3_set_step_replay",
               _lib().ikv_qwen3_set_step_replay(self._h, 1 if on else 0))

    def capture_logits(self, steps):
        """Keep the sampler's logits row at each of `steps` during later
        generate() calls (step 0: the prompt's last row; [] keeps none)."""
        st = np.ascontiguousarray(steps, dtype=np.int64)
        self._logit_steps = [int(x) for x in st]
        _check("ikv_qwen3_capture_logits",
               _lib().ikv_qwen3_capture_logits(self._h, st.ctypes.data if st.size else None,
                                               st.size))

    def captured_logits(self):
        """The kept rows of the last generate(): float32 [len(steps), n_vocab]."""
        n = len(self._logit_steps)
        out = np.empty((n, self.cfg.n_vocab), np.float32)
        _check("ikv_qwen3_captured_logits",
               _lib().ikv_qwen3_captured_logits(self._h, out.ctypes.data, out.size))
        return out

    def generate(self, prompt, n_gen: int):
        """Greedy tokens (list) and Timing for prompt then n_gen tokens."""
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(n_gen, np.int32)
        t = Timing()
        _check("ikv_qwen3_generate", _lib().ikv_qwen3_generate(
            self._h, p.ctypes.data, p.size, n_gen, out.ctypes.data, ctypes.byref(t)))
        return out.tolist(), t

    def generate_interleaved(self, prompts, n_gen: int):
        """Greedy tokens of several equal-length prompts decoded in turn (one
        step each per round): a list of token lists, and Timing per round."""
        p = np.ascontiguousarray(np.stack([np.asarray(x, np.int32) for x in prompts]))
        out = np.empty((p.shape[0], n_gen), np.int32)
        t = Timing()
        _check("ikv_qwen3_generate_interleaved", _lib().ikv_qwen3_generate_interleaved(
            self._h, p.ctypes.data, p.shape[0], p.shape[1], n_gen, out.ctypes.data,
            ctypes.byref(t)))
        return out.tolist(), t

    def last_stats(self):
        s = Stats()
        _check("ikv_qwen3_last_stats", _lib().ikv_qwen3_last_stats(self._h, ctypes.byref(s)))
        return {f: getattr(s, f) for f, _ in Stats._fields_}
