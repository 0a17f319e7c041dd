"""Pins for the oracle's ops around the path and its whole Qwen3 step
(oracle/oracle_model.c), on the CPU.

As for the hot-path ops, the reference holds no vectors for these (its only
known answers are model-level token checksums over the unavailable GGUF), so
each function is pinned by what the mathematics fixes: float64 brute force,
exact special cases (identity / one-hot products, copies), closed forms, and
the reference's own invariant that cached decode equals recomputing the whole
prefix (docs/performance/*/p*.csv hold identical token checksums for CPU
without and with the KV cache).
"""
import math

import numpy as np
import pytest

import oracle
from ikv import qwen3, synth

TINY = qwen3.Qwen3Config(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=128, n_ff=512,
                         n_vocab=1000, n_ctx_train=512)


@pytest.fixture(autouse=True, scope="module")
def _pool():
    oracle.set_workers(4)


def rms_f64(x, w, eps):
    x = x.astype(np.float64)
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * w.astype(np.float64)


def rope_f64(x, pos, theta):
    """NeoX rotation of x [n, H, D] by the table's angles at pos, in float64."""
    x = x.astype(np.float64)
    half = x.shape[-1] // 2
    a = theta[pos].astype(np.float64)[:, None, :]
    c, s = np.cos(a), np.sin(a)
    x0, x1 = x[..., :half], x[..., half:]
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)


def attn_f64(q, k, v, n_past):
    n_q, Hq, d = q.shape
    G = Hq // k.shape[1]
    kh, vh = np.repeat(k, G, axis=1), np.repeat(v, G, axis=1)
    s = np.einsum("thd,khd->htk", q, kh) / math.sqrt(d)
    mask = np.arange(k.shape[0])[None, :] > n_past + np.arange(n_q)[:, None]
    s = np.where(mask[None], -np.inf, s)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("htk,khd->thd", p, vh)


# ---------------------------------------------------------------------------
# mul_mat
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n_out,k,m", [(7, 5, 1), (64, 1024, 1), (33, 300, 4), (5, 3072, 2)])
def test_mul_mat_matches_float64(n_out, k, m):
    w = synth.normal(11 + k, (n_out, k))
    x = synth.normal(12 + k, (m, k))
    got = oracle.mul_mat(w, x)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    bound = 2e-6 * k * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T) + 1e-30
    assert np.all(np.abs(got - ref) <= bound)


def test_mul_mat_exact_cases():
    eye = np.eye(16, dtype=np.float32)
    x = synth.normal(3, (3, 16))
    assert np.array_equal(oracle.mul_mat(eye, x), x)            # identity
    w = synth.normal(4, (9, 16))
    onehot = np.zeros((2, 16), np.float32)
    onehot[0, 5] = 1.0
    onehot[1, 15] = 1.0
    got = oracle.mul_mat(w, onehot)
    assert np.array_equal(got[0], w[:, 5]) and np.array_equal(got[1], w[:, 15])  # columns, not rows


def test_mul_mat_is_the_sequential_float_sum():
    """One accumulator from 0.0f in index order: a case where pairwise or
    reversed summation rounds differently."""
    x = np.array([[1.0, 1e8, -1e8, 1.0]], np.float32)
    w = np.ones((1, 4), np.float32)
    # ((0 + 1) + 1e8) - 1e8 + 1 = 1 in float; a pairwise sum gives 2, reversed gives 0
    assert oracle.mul_mat(w, x)[0, 0] == np.float32(1.0)
    # the same rows as part of a multi-token product (the tiled loop nest)
    x4 = np.repeat(x, 5, axis=0)
    x4[1:, 0] = 2.0  # ((0 + 2) + 1e8) - 1e8 + 1 = 1 as well; reversed order gives 0
    assert np.all(oracle.mul_mat(np.repeat(w, 3, axis=0), x4) == np.float32(1.0))


@pytest.mark.parametrize("n_out,k,m", [(45, 1031, 37), (64, 1024, 4), (3, 7, 9), (96, 256, 64)])
def test_mul_mat_tiles_equal_per_token_products(n_out, k, m):
    """Products of four or more tokens run a tiled loop nest (32 outputs x 32
    tokens, four tokens per SSE chain); each element must keep the one-token
    path's bits (a sequential float sum), ragged tiles included."""
    w = synth.normal(51 + k, (n_out, k))
    x = synth.normal(52 + m, (m, k))
    got = oracle.mul_mat(w, x)
    for t in range(m):
        assert np.array_equal(got[t].view(np.uint32), oracle.mul_mat(w, x[t]).view(np.uint32))
    # and the one-token path is the sequential float32 sum
    seq = np.zeros(n_out, np.float32)
    for kk in range(k):
        seq = seq + x[m - 1, kk] * w[:, kk]
    assert np.array_equal(got[m - 1].view(np.uint32), seq.view(np.uint32))


# ---------------------------------------------------------------------------
# get_rows, elementwise, sampler
# ---------------------------------------------------------------------------

def test_get_rows_copies_rows_and_rejects_bad_ids():
    t = synth.normal(5, (50, 24))
    ids = np.array([0, 49, 7, 7], np.int32)
    assert np.array_equal(oracle.get_rows(t, ids), t[ids])
    with pytest.raises(ValueError):
        oracle.get_rows(t, np.array([50], np.int32))
    with pytest.raises(ValueError):
        oracle.get_rows(t, np.array([-1], np.int32))


def test_silu_closed_forms():
    x = synth.normal(6, (1000,)) * 4
    s = oracle.elementwise("silu", x)
    assert oracle.elementwise("silu", np.zeros(3, np.float32)).tolist() == [0.0, 0.0, 0.0]
    sm = oracle.elementwise("silu", -x)
    assert np.allclose(s.astype(np.float64) - sm, x, rtol=0, atol=2e-6 * (1 + np.abs(x)))
    ref = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    assert np.allclose(s, ref, rtol=3e-7, atol=1e-7)


def test_add_mul_exact():
    a, b = synth.normal(7, (100,)), synth.normal(8, (100,))
    assert np.array_equal(oracle.elementwise("add", a, b), a + b)
    assert np.array_equal(oracle.elementwise("mul", a, b), a * b)


def test_sample_greedy_rules():
    assert oracle.sample_greedy(np.array([1, 3, 3, 2], np.float32)) == 1      # tie -> lowest id
    assert oracle.sample_greedy(np.array([-np.inf, -5], np.float32)) == 1
    assert oracle.sample_greedy(np.array([0, np.nan, 9], np.float32)) == -1   # NaN rejected
    assert oracle.sample_greedy(np.array([0, np.inf], np.float32)) == -1      # +inf rejected
    assert oracle.sample_greedy(np.array([-np.inf, -np.inf], np.float32)) == -1
    x = synth.normal(9, (151936,))
    assert oracle.sample_greedy(x) == int(np.argmax(x))


# ---------------------------------------------------------------------------
# the whole step
# ---------------------------------------------------------------------------

def step_f64(cfg, w, tokens, n_past, kc, vc, theta):
    """float64 restatement of one Qwen3 step from the graph in
    src/models/Qwen3.cpp:4-136 (independent of the oracle's C code)."""
    n = len(tokens)
    D, Hq, Hkv = cfg.head_dim, cfg.n_head, cfg.n_head_kv
    f = lambda a: a.astype(np.float64)
    x = f(w["token_embd.weight"])[tokens]
    pos = np.arange(n_past, n_past + n)
    for i in range(cfg.n_layer):
        p = f"blk.{i}."
        cur = rms_f64(x, w[p + "attn_norm.weight"], cfg.rms_norm_eps)
        q = (cur @ f(w[p + "attn_q.weight"]).T).reshape(n, Hq, D)
        k = (cur @ f(w[p + "attn_k.weight"]).T).reshape(n, Hkv, D)
        v = (cur @ f(w[p + "attn_v.weight"]).T).reshape(n, Hkv, D)
        q = rope_f64(rms_f64(q, w[p + "attn_q_norm.weight"], cfg.rms_norm_eps), pos, theta)
        k = rope_f64(rms_f64(k, w[p + "attn_k_norm.weight"], cfg.rms_norm_eps), pos, theta)
        kc[i][n_past:n_past + n] = k
        vc[i][n_past:n_past + n] = v
        a = attn_f64(q, kc[i][:n_past + n], vc[i][:n_past + n], n_past).reshape(n, Hq * D)
        ffn_inp = a @ f(w[p + "attn_output.weight"]).T + x
        cur = rms_f64(ffn_inp, w[p + "ffn_norm.weight"], cfg.rms_norm_eps)
        g = cur @ f(w[p + "ffn_gate.weight"]).T
        u = cur @ f(w[p + "ffn_up.weight"]).T
        x = (u * (g / (1 + np.exp(-g)))) @ f(w[p + "ffn_down.weight"]).T + ffn_inp
    x = rms_f64(x, w["output_norm.weight"], cfg.rms_norm_eps)
    return x @ f(w["token_embd.weight"]).T


def tiny_weights(seed=0x1F0000 + 99):
    w = qwen3.synthetic_weights(TINY, seed, std=0.05)
    for name in w:  # norm weights away from 1 so that a dropped weight shows
        if "norm" in name:
            w[name] = (1.0 + 0.3 * synth.normal(hash(name) & 0xFFFF, w[name].shape)).astype(np.float32)
    return w


def test_qwen3_step_matches_float64_model():
    w = tiny_weights()
    cap = 40
    orc = oracle.Qwen3Oracle(TINY, w, cap)
    theta = orc.theta
    kc = [np.zeros((cap, TINY.n_head_kv, TINY.head_dim)) for _ in range(TINY.n_layer)]
    vc = [np.zeros_like(a) for a in kc]
    tokens = synth.uniform_ints(3, 9, TINY.n_vocab)
    got = orc.step(tokens, 0, last_row_only=False)
    ref = step_f64(TINY, w, tokens, 0, kc, vc, theta)
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
    # then two decode steps against the same float64 caches
    n_past = len(tokens)
    for t in (5, 999):
        got = orc.step([t], n_past)
        ref = step_f64(TINY, w, [t], n_past, kc, vc, theta)
        assert np.allclose(got[-1], ref[-1], rtol=1e-4, atol=1e-4 * np.abs(ref).max())
        n_past += 1


def test_qwen3_cached_decode_equals_recompute_bitwise():
    """Logits of step-by-step decode equal the rows of one prefill over the
    same tokens, bit for bit (rows are independent except attention, whose
    masked keys add exact zeros)."""
    w = tiny_weights(7)
    tokens = synth.uniform_ints(4, 12, TINY.n_vocab)
    full = oracle.Qwen3Oracle(TINY, w, 16).step(tokens, 0, last_row_only=False)
    inc = oracle.Qwen3Oracle(TINY, w, 16)
    rows = [inc.step(tokens[:5], 0, last_row_only=False)]
    for i in range(5, len(tokens)):
        rows.append(inc.step(tokens[i:i + 1], i))
    assert np.array_equal(np.concatenate(rows).view(np.uint32), full.view(np.uint32))


def test_qwen3_generate_is_greedy_over_steps():
    w = tiny_weights(8)
    orc = oracle.Qwen3Oracle(TINY, w, 32)
    prompt = synth.uniform_ints(5, 6, TINY.n_vocab)
    toks = orc.generate(prompt, 8)
    ref = oracle.Qwen3Oracle(TINY, w, 32)
    ids = list(prompt)
    for i, tok in enumerate(toks):
        logits = ref.step(ids, 0, last_row_only=False)   # recompute the whole prefix
        assert tok == oracle.sample_greedy(logits[-1]), i
        ids.append(tok)
        ref = oracle.Qwen3Oracle(TINY, w, 32)
