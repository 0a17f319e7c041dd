"""GPU parity of the ops around the KV-cache path and of the whole Qwen3 model
on the HIP backend, against the oracle (restated reference CPU backend).

Bars: gathers, adds, products and the sampler bit-exact; projections within
1e-4 of sum_k |x_k w_k| (an F32 dot product in another summation order; a
dropped or misplaced term is ~1/K of that sum, above the bar for K <= 4096);
silu within 1e-6 relative; the model: identical greedy token streams.
"""
import numpy as np
import pytest

import ikv
import oracle
from ikv import qwen3, synth

pytestmark = pytest.mark.gpu


def dev_t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def proj_close(got, w, x, ref):
    scale = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    return np.all(np.abs(got.astype(np.float64) - ref) <= 1e-4 * scale + 1e-30)


# ---------------------------------------------------------------------------
# projections
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n_out,k", [(2048, 1024), (1024, 2048), (1024, 3072), (3072, 1024),
                                     (151936, 1024), (4096, 4096), (100, 1000), (7, 64)])
def test_gemv_matches_oracle(dev, oracle_pool, n_out, k):
    w = synth.normal(100 + n_out, (n_out, k), 0.02)
    x = synth.normal(200 + k, (k,))
    got = host(ikv.mul_mat(dev_t(w, dev), dev_t(x, dev)))
    assert proj_close(got, w, x[None], oracle.mul_mat(w, x))


@pytest.mark.parametrize("n_out,k,m", [(2048, 1024, 37), (1024, 3072, 5), (300, 200, 2)])
def test_mul_mat_multi_token_matches_oracle(dev, oracle_pool, n_out, k, m):
    w = synth.normal(300 + m, (n_out, k), 0.02)
    x = synth.normal(400 + m, (m, k))
    r = synth.normal(500 + m, (m, n_out))
    got = host(ikv.mul_mat(dev_t(w, dev), dev_t(x, dev)))
    assert proj_close(got, w, x, oracle.mul_mat(w, x))
    got_r = host(ikv.mul_mat(dev_t(w, dev), dev_t(x, dev), residual=dev_t(r, dev)))
    assert proj_close(got_r, w, x, oracle.mul_mat(w, x).astype(np.float64) + r)


def test_gemv_residual_in_place(dev, oracle_pool):
    w = synth.normal(7, (1024, 2048), 0.02)
    x = synth.normal(8, (2048,))
    r = synth.normal(9, (1024,))
    rd = dev_t(r, dev)
    ikv.mul_mat(dev_t(w, dev), dev_t(x, dev), out=rd, residual=rd)
    assert proj_close(host(rd), w, x[None], oracle.mul_mat(w, x).astype(np.float64) + r)


def test_gemv3_equals_three_projections(dev, oracle_pool):
    x = synth.normal(10, (1024,))
    ws = [synth.normal(11 + i, (n, 1024), 0.02) for i, n in enumerate((2048, 1024, 1024))]
    outs = ikv.gemv3(*[dev_t(w, dev) for w in ws], dev_t(x, dev))
    for w, o in zip(ws, outs):
        assert proj_close(host(o), w, x[None], oracle.mul_mat(w, x))


@pytest.mark.parametrize("n_out,k", [(3072, 1024), (12288, 4096), (50, 100)])
def test_gemv_swiglu_matches_oracle(dev, oracle_pool, n_out, k):
    wg = synth.normal(12, (n_out, k), 0.05)
    wu = synth.normal(13, (n_out, k), 0.05)
    x = synth.normal(14, (k,))
    got = host(ikv.gemv_swiglu(dev_t(wg, dev), dev_t(wu, dev), dev_t(x, dev))).astype(np.float64)
    g = oracle.mul_mat(wg, x)
    u = oracle.mul_mat(wu, x)
    ref = oracle.elementwise("mul", u, oracle.elementwise("silu", g)).astype(np.float64)
    # error of the two dots, propagated through u * silu(g) (|silu'| <= 1.1)
    sg = np.abs(x.astype(np.float64)) @ np.abs(wg.astype(np.float64)).T
    su = np.abs(x.astype(np.float64)) @ np.abs(wu.astype(np.float64)).T
    silu_g = np.abs(oracle.elementwise("silu", g).astype(np.float64))
    bound = 1e-4 * (su * silu_g + 1.1 * np.abs(u) * sg) + 1e-6 * np.abs(ref) + 1e-30
    assert np.all(np.abs(got - ref) <= bound)


# ---------------------------------------------------------------------------
# small ops
# ---------------------------------------------------------------------------

def test_get_rows_bit_exact_and_bad_id_zeroed(dev):
    import torch
    t = synth.normal(15, (1000, 1024))
    ids = np.array([0, 999, 17, 17, 500], np.int32)
    got = host(ikv.get_rows(dev_t(t, dev), dev_t(ids, dev)))
    assert np.array_equal(got.view(np.uint32), t[ids].view(np.uint32))
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    bad = np.array([3, 1000, -1], np.int32)
    got = host(ikv.get_rows(dev_t(t, dev), dev_t(bad, dev), status=status))
    assert np.array_equal(got[0], t[3]) and not got[1:].any()
    assert int(host(status)[0]) == 1


@pytest.mark.parametrize("n", [1, 1000, 3072, 4097])
def test_elementwise(dev, n):
    a, b = synth.normal(16 + n, (n,)) * 3, synth.normal(17 + n, (n,))
    da, db = dev_t(a, dev), dev_t(b, dev)
    assert np.array_equal(host(ikv.elementwise("add", da, db)), oracle.elementwise("add", a, b))
    assert np.array_equal(host(ikv.elementwise("mul", da, db)), oracle.elementwise("mul", a, b))
    assert np.allclose(host(ikv.elementwise("silu", da)), oracle.elementwise("silu", a),
                       rtol=1e-6, atol=1e-7)


def test_argmax_follows_the_greedy_sampler(dev):
    import torch
    x = synth.normal(18, (151936,))
    assert int(host(ikv.argmax(dev_t(x, dev)))[0]) == oracle.sample_greedy(x)
    y = x.copy()
    y[[5, 70000, 151935]] = 100.0                       # tie: lowest id wins
    assert int(host(ikv.argmax(dev_t(y, dev)))[0]) == 5 == oracle.sample_greedy(y)
    for bad in (np.nan, np.inf):
        z = x.copy()
        z[1234] = bad
        assert int(host(ikv.argmax(dev_t(z, dev)))[0]) == -1 == oracle.sample_greedy(z)
    ninf = np.full(1000, -np.inf, np.float32)
    assert int(host(ikv.argmax(dev_t(ninf, dev)))[0]) == -1
    # unaligned start (scalar path) and a short odd length
    big = dev_t(np.concatenate([[0.0], y]).astype(np.float32), dev)
    assert int(host(ikv.argmax(big[1:]))[0]) == 5
    w = synth.normal(19, (7,))
    assert int(host(ikv.argmax(dev_t(w, dev)))[0]) == int(np.argmax(w))
    del torch


# ---------------------------------------------------------------------------
# the whole model
# ---------------------------------------------------------------------------

SMALL = qwen3.Qwen3Config(n_layer=4, n_vocab=8192, n_ctx_train=4096)


def engine_with(cfg, weights, max_ctx):
    eng = qwen3.Qwen3Engine(cfg, max_ctx)
    eng.set_weights(weights)
    return eng


def test_small_model_greedy_tokens_match_oracle(dev, oracle_pool):
    w = qwen3.synthetic_weights(SMALL, synth.config_seed(0, 10))
    prompt = synth.uniform_ints(synth.config_seed(0, 11), 32, SMALL.n_vocab)
    eng = engine_with(SMALL, w, 128)
    toks, t = eng.generate(prompt, 48)
    stats = eng.last_stats()
    ref = oracle.Qwen3Oracle(SMALL, w, 128).generate(prompt, 48)
    assert toks == ref
    # a decode step took every fusion: per layer qk-norm+RoPE x2, append+decode,
    # q/k/v, SwiGLU, o_proj+residual and down+residual
    L = SMALL.n_layer
    assert stats["fused_norm_rope"] == 2 * L and stats["fused_append_decode"] == L
    assert stats["fused_qkv"] == L and stats["fused_swiglu"] == L and stats["fused_residual"] == 2 * L
    assert t.ttft_s > 0 and t.tpot_s > 0
    # unfused graph (every node its own kernel) gives the same tokens
    eng.set_fusion(False)
    assert eng.generate(prompt, 48)[0] == ref
    eng.close()


def test_synthetic_init_on_device_equals_host_weights(dev):
    w = qwen3.synthetic_weights(SMALL, 0x5EED)
    prompt = synth.uniform_ints(3, 20, SMALL.n_vocab)
    a = engine_with(SMALL, w, 64)
    b = qwen3.Qwen3Engine(SMALL, 64)
    b.init_synthetic(0x5EED)
    assert a.tensor_names() == [n for n, _ in qwen3.tensor_layout(SMALL)]
    assert a.generate(prompt, 16)[0] == b.generate(prompt, 16)[0]
    a.close()
    b.close()


def test_qwen3_06b_config0_greedy_tokens_match_oracle(dev, oracle_pool):
    """Qwen3-0.6B architecture F32, random init (std 0.02,
    norms 1.0), 32 uniform prompt ids, 128 greedy steps, no EOS stop."""
    cfg = qwen3.QWEN3_0_6B
    w = qwen3.synthetic_weights(cfg, synth.config_seed(0, 1))
    prompt = synth.uniform_ints(synth.config_seed(0, 0), 32, cfg.n_vocab)
    eng = engine_with(cfg, w, 160)
    toks, _ = eng.generate(prompt, 128)
    eng.close()
    ref = oracle.Qwen3Oracle(cfg, w, 160).generate(prompt, 128)
    assert toks == ref
