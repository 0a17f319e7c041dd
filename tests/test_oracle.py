"""Pins for the CPU oracle (oracle/oracle.c), the checker of the HIP path.

The reference holds no op-level golden vectors (its only known answers are
model-level token checksums that need the unavailable Qwen3-0.6B GGUF), so the
oracle is pinned by what the mathematics fixes: float64 brute force, closed
forms and invariants, each chosen so that a plausible slip (wrong pairing, GQA
mapping, mask offset, scale, accumulation precision) fails at least one.
"""
import numpy as np
import pytest

import oracle
from ikv import synth

D = 128


@pytest.fixture(autouse=True, scope="module")
def _pool():
    oracle.set_workers(4)


# ---------------------------------------------------------------------------
# float64 references written independently of the oracle (vectorised numpy)
# ---------------------------------------------------------------------------

def attn_f64(q, k, v, n_past):
    q = q.astype(np.float64)
    k = k.astype(np.float64)
    v = v.astype(np.float64)
    n_q, Hq, d = q.shape
    n_kv, Hkv, _ = k.shape
    G = Hq // Hkv
    kh = np.repeat(k, G, axis=1)  # [n_kv, Hq, d]: q head h -> kv head h // G
    vh = np.repeat(v, G, axis=1)
    s = np.einsum("thd,khd->htk", q, kh) / np.sqrt(d)
    t = np.arange(n_q)[:, None]
    kk = np.arange(n_kv)[None, :]
    s = np.where((kk > n_past + t)[None], -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("htk,khd->thd", p, vh)


def rms_f64(x, w, eps):
    x = x.astype(np.float64)
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * w.astype(np.float64)


def close(a, b, rtol, atol):
    err = np.abs(a.astype(np.float64) - b.astype(np.float64))
    return bool(np.all(err <= atol + rtol * np.abs(b.astype(np.float64))))


# ---------------------------------------------------------------------------
# RMS norm
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("rows,dim", [(1, 128), (24, 128), (5, 1024), (3, 7)])
def test_rms_norm_matches_float64(rows, dim):
    x = synth.normal(11 + dim, (rows, dim))
    w = synth.normal(12 + dim, (dim,))
    got = oracle.rms_norm(x, w, 1e-6)
    assert close(got, rms_f64(x, w, 1e-6), 2e-6, 1e-6)


def test_rms_norm_unit_weight_has_unit_rms():
    x = synth.normal(13, (16, 128), std=3.0)
    got = oracle.rms_norm(x, np.ones(128, np.float32), 1e-6).astype(np.float64)
    assert np.allclose(np.sqrt((got * got).mean(axis=-1)), 1.0, rtol=1e-6)


def test_rms_norm_rounding_points():
    """Float squares summed in double in index order, scale rounded to float,
    then (x*scale)*w in float (cpu_backend.cpp:369-378). A double-precision
    product, a float accumulator or x*(scale*w) would differ in some rows."""
    x = synth.normal(14, (64, 128), std=5.0)
    w = synth.normal(15, (128,))
    sq = (x * x).astype(np.float64)
    s = np.cumsum(sq, axis=1)[:, -1]  # sequential double sum
    scale = (1.0 / np.sqrt(s / 128 + np.float64(np.float32(1e-6)))).astype(np.float32)
    want = (x * scale[:, None]).astype(np.float32) * w
    got = oracle.rms_norm(x, w, 1e-6)
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


# ---------------------------------------------------------------------------
# RoPE angle table and rotation
# ---------------------------------------------------------------------------

def test_theta_table_closed_form():
    th = oracle.rope_theta_table(1e6, D, 4096)
    pos = np.arange(4096, dtype=np.float64)[:, None]
    i = np.arange(D // 2, dtype=np.float64)[None, :]
    want = pos * 1e6 ** (-2.0 * i / D)
    assert np.all(th[0] == 0.0)
    assert np.array_equal(th[:, 0], np.arange(4096, dtype=np.float32))  # freq_0 == 1
    assert close(th, want, 2e-6, 0.0)


def test_rope_position_zero_is_identity():
    x = synth.normal(21, (2, 3, D))
    th = oracle.rope_theta_table(1e6, D, 8)
    got = oracle.rope_neox(x, np.zeros(2, np.int32), th)
    assert np.array_equal(got, x)


def test_rope_matches_float64_neox_rotation():
    x = synth.normal(22, (5, 4, D))
    pos = np.array([1, 7, 100, 4095, 2], np.int32)
    th = oracle.rope_theta_table(1e6, D, 4096)
    got = oracle.rope_neox(x, pos, th)
    a = th[pos].astype(np.float64)[:, None, :]  # angles used by the op
    x0 = x[..., : D // 2].astype(np.float64)
    x1 = x[..., D // 2:].astype(np.float64)
    want = np.concatenate([x0 * np.cos(a) - x1 * np.sin(a), x0 * np.sin(a) + x1 * np.cos(a)], -1)
    assert close(got, want, 1e-5, 1e-6)
    # each (j, j+D/2) pair keeps its length
    n_in = np.hypot(x0, x1)
    n_out = np.hypot(got[..., : D // 2].astype(np.float64), got[..., D // 2:].astype(np.float64))
    assert np.allclose(n_in, n_out, rtol=1e-6, atol=1e-7)


def test_rope_rejects_out_of_table_position():
    th = oracle.rope_theta_table(1e6, D, 8)
    with pytest.raises(ValueError):
        oracle.rope_neox(np.zeros((1, 1, D), np.float32), np.array([8], np.int32), th)


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n_q,n_kv,n_past,Hq,Hkv", [
    (1, 1, 0, 16, 8), (1, 257, 256, 16, 8), (1, 1025, 1024, 32, 8), (7, 7, 0, 16, 8),
    (5, 12, 7, 16, 8), (33, 33, 0, 8, 8), (4, 20, 16, 16, 2),
])
def test_attention_matches_float64(n_q, n_kv, n_past, Hq, Hkv):
    q = synth.normal(31, (n_q, Hq, D))
    k = synth.normal(32, (n_kv, Hkv, D))
    v = synth.normal(33, (n_kv, Hkv, D))
    got = oracle.flash_attn(q, k, v, n_past)
    assert close(got, attn_f64(q, k, v, n_past), 1e-5, 1e-6)


def test_attention_single_key_returns_its_value():
    q = synth.normal(34, (1, 16, D))
    k = synth.normal(35, (1, 8, D))
    v = synth.normal(36, (1, 8, D))
    got = oracle.flash_attn(q, k, v, 0)
    assert np.array_equal(got[0], np.repeat(v[0], 2, axis=0))


def test_attention_identical_keys_average_values():
    q = synth.normal(37, (1, 16, D))
    k = np.repeat(synth.normal(38, (1, 8, D)), 50, axis=0)
    v = synth.normal(39, (50, 8, D))
    got = oracle.flash_attn(q, k, v, 49)
    assert close(got[0], np.repeat(v.astype(np.float64).mean(0), 2, axis=0), 1e-5, 1e-6)


def test_attention_aligned_key_dominates():
    k = synth.normal(40, (64, 8, D))
    v = synth.normal(41, (64, 8, D))
    q = np.repeat(k[17:18] * 40.0, 2, axis=1)  # q head 2g, 2g+1 aligned with key 17 of head g
    got = oracle.flash_attn(q, k, v, 63)
    assert close(got[0], np.repeat(v[17], 2, axis=0), 1e-4, 1e-4)


def test_attention_gqa_head_mapping_by_permutation():
    q = synth.normal(42, (3, 16, D))
    k = synth.normal(43, (3, 8, D))
    v = synth.normal(44, (3, 8, D))
    perm = np.array([3, 0, 7, 1, 6, 2, 5, 4])
    qperm = np.concatenate([np.arange(2 * p, 2 * p + 2) for p in perm])
    a = oracle.flash_attn(q, k, v, 0)
    b = oracle.flash_attn(q[:, qperm], k[:, perm], v[:, perm], 0)
    assert np.array_equal(a[:, qperm], b)


def test_attention_causal_future_key_has_no_effect():
    q = synth.normal(45, (6, 16, D))
    k = synth.normal(46, (6, 8, D))
    v = synth.normal(47, (6, 8, D))
    a = oracle.flash_attn(q, k, v, 0)
    k2, v2 = k.copy(), v.copy()
    k2[5] += 3.0
    v2[5] -= 7.0
    b = oracle.flash_attn(q, k2, v2, 0)
    assert np.array_equal(a[:5], b[:5]) and not np.array_equal(a[5], b[5])


def test_attention_decode_steps_equal_prefill_rows():
    """Cached decode equals recompute: row t of a prefill over P tokens is the
    decode of token t over keys [0, t] (the reference-held invariant of its
    identical CPU-no-KV / CPU-KV token checksums)."""
    P = 40
    q = synth.normal(48, (P, 16, D))
    k = synth.normal(49, (P, 8, D))
    v = synth.normal(50, (P, 8, D))
    full = oracle.flash_attn(q, k, v, 0)
    for t in (0, 1, 17, 39):
        step = oracle.flash_attn(q[t:t + 1], k[: t + 1], v[: t + 1], t)
        assert np.array_equal(step[0], full[t])


# ---------------------------------------------------------------------------
# append
# ---------------------------------------------------------------------------

def test_cpy_and_decode_append_write_only_the_new_row():
    cap, L = 20, 9
    k_cache = np.full((cap, 8, D), np.float32(-1234.5), np.float32)
    v_cache = np.full((cap, 8, D), np.float32(4321.0), np.float32)
    k_hist = synth.normal(51, (L, 8, D))
    v_hist = synth.normal(52, (L, 8, D))
    oracle.cpy(k_cache[:L], k_hist)
    oracle.cpy(v_cache[:L], v_hist)
    kn = synth.normal(53, (8, D))
    vn = synth.normal(54, (8, D))
    q = synth.normal(55, (16, D))
    out = oracle.decode_append_attn(q, kn, vn, k_cache, v_cache, L)
    assert np.array_equal(k_cache[:L], k_hist) and np.array_equal(k_cache[L], kn)
    assert np.all(k_cache[L + 1:] == np.float32(-1234.5))
    assert np.array_equal(v_cache[L], vn) and np.all(v_cache[L + 1:] == np.float32(4321.0))
    k_all = np.concatenate([k_hist, kn[None]])
    v_all = np.concatenate([v_hist, vn[None]])
    assert close(out, attn_f64(q[None], k_all, v_all, L)[0], 1e-5, 1e-6)


def test_worker_count_does_not_change_results():
    q = synth.normal(56, (9, 16, D))
    k = synth.normal(57, (30, 8, D))
    v = synth.normal(58, (30, 8, D))
    oracle.set_workers(1)
    a = oracle.flash_attn(q, k, v, 21)
    oracle.set_workers(6)
    b = oracle.flash_attn(q, k, v, 21)
    assert np.array_equal(a, b)
