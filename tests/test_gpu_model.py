"""GPU parity of the ops around the KV-cache path and of the whole Qwen3 model
on the HIP backend, against the oracle (restated reference CPU backend).

Bars: gathers, adds, products and the sampler bit-exact; projections within
1e-4 of sum_k |x_k w_k| (an F32 dot product in another summation order; a
dropped or misplaced term is ~1/K of that sum, above the bar for K <= 4096);
silu within 1e-6 relative; the model: identical greedy token streams.
"""
import errno

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


@pytest.mark.parametrize("n_out,k,m", [(2048, 1024, 37), (1024, 3072, 5), (300, 200, 2), (3072, 1024, 64),
                                        (16, 256, 2), (4096, 4096, 17), (1024, 2048, 65),
                                        (2048, 1024, 300), (3072, 1024, 2048), (1024, 3072, 129),
                                        (4096, 4096, 100), (192, 64, 70), (300, 200, 100),
                                        (4096, 1024, 64), (4096, 2048, 40),  # two token tiles per workgroup
                                        (96, 200, 2100), (1024, 1024, 1000), (4096, 1024, 512)])
def test_mul_mat_multi_token_matches_oracle(dev, oracle_pool, n_out, k, m):
    w = synth.normal(300 + m, (n_out, k), 0.02)
    x = synth.normal(400 + m, (m, k))
    r = synth.normal(500 + m, (m, n_out))
    got = host(ikv.mul_mat(dev_t(w, dev), dev_t(x, dev)))
    assert proj_close(got, w, x, oracle.mul_mat(w, x))
    got_r = host(ikv.mul_mat(dev_t(w, dev), dev_t(x, dev), residual=dev_t(r, dev)))
    assert proj_close(got_r, w, x, oracle.mul_mat(w, x).astype(np.float64) + r)


def test_mul_mat_few_tokens_residual_in_place(dev, oracle_pool):
    # out = out + W x for a 32-token batch (the few-token MFMA path)
    n_out, k, m = 1024, 2048, 32
    w = synth.normal(610, (n_out, k), 0.02)
    x = synth.normal(611, (m, k))
    r = synth.normal(612, (m, n_out))
    buf = dev_t(r, dev)
    ikv.mul_mat(dev_t(w, dev), dev_t(x, dev), out=buf, residual=buf)
    assert proj_close(host(buf), w, x, oracle.mul_mat(w, x).astype(np.float64) + r)


def test_mul_mat_many_tokens_residual_in_place(dev, oracle_pool):
    # out = out + W x through the MFMA GEMM: 65 tokens (K split in two), 200
    # and 2048
    for m in (65, 200, 2048):
        _many_tokens_residual_in_place(dev, m)


def _many_tokens_residual_in_place(dev, m):
    n_out, k = 1024, 2048
    w = synth.normal(620, (n_out, k), 0.02)
    x = synth.normal(621, (m, k))
    r = synth.normal(622, (m, n_out))
    buf = dev_t(r, dev)
    ikv.mul_mat(dev_t(w, dev), dev_t(x, dev), out=buf, residual=buf)
    assert proj_close(host(buf), w, x, oracle.mul_mat(w, x).astype(np.float64) + r)


@pytest.mark.parametrize("n_out,k,m", [
    (128, 64, 1), (192, 128, 65), (1024, 256, 200), (256, 2048, 129),  # 64 x 64 tiles, ragged m
    (8192, 64, 2048), (8192, 128, 2047), (8192, 64, 2100),             # 128 x 128 tiles (>= 4 rounds)
    (3072, 1024, 2048),                                               # a Qwen3-0.6B prefill shape
])
def test_gemm_matches_oracle(dev, oracle_pool, n_out, k, m):
    # the MFMA GEMM through its own entry, at token counts below the mul_mat
    # threshold too; both tile shapes and tokens past the last whole tile
    w = synth.normal(700 + m, (n_out, k), 0.02)
    x = synth.normal(701 + m, (m, k))
    r = synth.normal(702 + m, (m, n_out))
    ref = oracle.mul_mat(w, x)
    got = host(ikv.gemm_nt(dev_t(w, dev), dev_t(x, dev)))
    assert proj_close(got, w, x, ref)
    buf = dev_t(r, dev)
    ikv.gemm_nt(dev_t(w, dev), dev_t(x, dev), out=buf, residual=buf)
    assert proj_close(host(buf), w, x, ref.astype(np.float64) + r)


@pytest.mark.parametrize("n_out,k,m", [(1024, 256, 200), (8192, 128, 2047)])
def test_gemm_unaligned_output_equals_aligned(dev, n_out, k, m):
    # an output or residual that is not 16-byte aligned takes the 4-byte
    # stores of the output tile: the same values, bit for bit
    import torch
    w = dev_t(synth.normal(710 + m, (n_out, k), 0.02), dev)
    x = dev_t(synth.normal(711 + m, (m, k)), dev)
    r = synth.normal(712 + m, (m, n_out))
    want = ikv.gemm_nt(w, x)
    want_r = ikv.gemm_nt(w, x, residual=dev_t(r, dev))
    buf = torch.empty(m * n_out + 1, device=dev)
    got = buf[1:].view(m, n_out)
    ikv.gemm_nt(w, x, out=got)
    assert torch.equal(got, want)
    got.copy_(dev_t(r, dev))
    ikv.gemm_nt(w, x, out=got, residual=got)
    assert torch.equal(got, want_r)


def gemm_plan(n_out, k, m):
    import ctypes
    tile, split = ctypes.c_int(), ctypes.c_int()
    assert ikv.load_bench().ikv_bench_gemm_plan(n_out, k, m, ctypes.byref(tile),
                                                ctypes.byref(split)) == 0
    return tile.value, split.value


@pytest.mark.parametrize("n_out,k,m", [
    (1024, 4096, 128), (1024, 3072, 128), (1024, 1024, 65),  # Qwen3 o / down / k,v shapes
    (64, 4096, 300), (128, 2048, 77), (192, 1600, 40),       # ragged m and k ranges
])
def test_mul_mat_split_k_matches_oracle(dev, oracle_pool, n_out, k, m):
    # tiles that leave CUs idle: each tile's K range split over several
    # workgroups, partials added in split order by the last to finish
    assert gemm_plan(n_out, k, m)[1] > 1
    w = synth.normal(800 + m, (n_out, k), 0.02)
    x = synth.normal(801 + m, (m, k))
    r = synth.normal(802 + m, (m, n_out))
    ref = oracle.mul_mat(w, x)
    wd, xd = dev_t(w, dev), dev_t(x, dev)
    got = host(ikv.mul_mat(wd, xd))
    assert proj_close(got, w, x, ref)
    for _ in range(3):  # deterministic, and every tile counter back at 0
        assert np.array_equal(host(ikv.mul_mat(wd, xd)), got)
    buf = dev_t(r, dev)
    ikv.mul_mat(wd, xd, out=buf, residual=buf)
    assert proj_close(host(buf), w, x, ref.astype(np.float64) + r)


@pytest.mark.parametrize("tile", range(5))
def test_gemm_every_tile_and_split_matches_oracle(dev, oracle_pool, tile):
    # each tile shape with K in 1, 2, 3, 5 and 8 ranges (25 steps of 64
    # columns: uneven ranges), ragged m, residual in place, through the
    # bench library's entry (the plan picks among these)
    import ctypes
    import torch
    n_out, k, m = 256, 1600, 77
    w = synth.normal(820 + tile, (n_out, k), 0.02)
    x = synth.normal(821 + tile, (m, k))
    r = synth.normal(822 + tile, (m, n_out))
    ref = oracle.mul_mat(w, x)
    wd, xd = dev_t(w, dev), dev_t(x, dev)
    ws = torch.zeros((16 << 10) + (4 << 20), dtype=torch.uint8, device=dev)
    lib = ikv.load_bench()
    stream = torch.cuda.current_stream().cuda_stream
    for split in (1, 2, 3, 5, 8):
        out = torch.empty(m, n_out, device=dev)
        assert lib.ikv_bench_gemm_nt_tile_f32(wd.data_ptr(), xd.data_ptr(), out.data_ptr(), n_out, k,
                                              m, None, tile, split, ws.data_ptr(), ws.numel(),
                                              stream) == 0
        assert proj_close(host(out), w, x, ref), f"tile {tile} split {split}"
        buf = dev_t(r, dev)
        assert lib.ikv_bench_gemm_nt_tile_f32(wd.data_ptr(), xd.data_ptr(), buf.data_ptr(), n_out, k,
                                              m, buf.data_ptr(), tile, split, ws.data_ptr(),
                                              ws.numel(), stream) == 0
        assert proj_close(host(buf), w, x, ref.astype(np.float64) + r), f"tile {tile} split {split}"
    torch.cuda.synchronize()
    assert not ws[:16 << 10].any()  # every tile counter back at 0


def test_mul_mat_split_k_replays_from_a_graph(dev):
    # the split-K product captured in a HIP graph (its stream's workspace
    # allocated by an eager call first): every replay equals the eager bits
    import torch
    w = dev_t(synth.normal(810, (1024, 2048), 0.02), dev)
    x = dev_t(synth.normal(811, (128, 2048)), dev)
    assert gemm_plan(1024, 2048, 128)[1] > 1
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    out = torch.empty(128, 1024, device=dev)
    with torch.cuda.stream(side):
        ikv.mul_mat(w, x, out=out)
    torch.cuda.synchronize()
    ref = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        ikv.mul_mat(w, x, out=out)
        ikv.mul_mat(w, x, out=out)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        ikv.mul_mat(w, x, out=out)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, ref)


def test_gemm_is_deterministic_and_mul_mat_uses_it(dev):
    # at 2048 tokens mul_mat runs the GEMM: same bits as the direct entry,
    # and the same bits on every call
    w = dev_t(synth.normal(710, (1024, 1024), 0.02), dev)
    x = dev_t(synth.normal(711, (2048, 1024)), dev)
    a = host(ikv.gemm_nt(w, x))
    assert np.array_equal(a, host(ikv.gemm_nt(w, x)))
    assert np.array_equal(a, host(ikv.mul_mat(w, x)))


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
    assert int(host(status)[0]) == ikv.STATUS_TOKEN


@pytest.mark.parametrize("n", [1, 1000, 3072, 4097])
def test_elementwise(dev, n):
    a, b = synth.normal(16 + n, (n,)) * 3, synth.normal(17 + n, (n,))
    da, db = dev_t(a, dev), dev_t(b, dev)
    assert np.array_equal(host(ikv.elementwise("add", da, db)), oracle.elementwise("add", a, b))
    assert np.array_equal(host(ikv.elementwise("mul", da, db)), oracle.elementwise("mul", a, b))
    assert np.allclose(host(ikv.elementwise("silu", da)), oracle.elementwise("silu", a),
                       rtol=1e-6, atol=1e-7)
    # up * silu(gate) in one pass equals SILU then MUL bit for bit (in place too)
    sep = host(ikv.elementwise("mul", db, ikv.elementwise("silu", da)))
    assert np.array_equal(host(ikv.elementwise("silu_mul", da, db)).view(np.uint32), sep.view(np.uint32))
    inplace = da.clone()
    ikv.elementwise("silu_mul", inplace, db, out=inplace)
    assert np.array_equal(host(inplace).view(np.uint32), sep.view(np.uint32))


@pytest.mark.parametrize("form", ["one_workgroup", "workspace"])
def test_argmax_follows_the_greedy_sampler(dev, form):
    import torch
    ws = ikv.argmax_workspace(dev) if form == "workspace" else None  # shared by every call below
    x = synth.normal(18, (151936,))
    assert int(host(ikv.argmax(workspace=ws, logits=dev_t(x, dev)))[0]) == oracle.sample_greedy(x)
    y = x.copy()
    y[[5, 70000, 151935]] = 100.0                       # tie: lowest id wins
    assert int(host(ikv.argmax(workspace=ws, logits=dev_t(y, dev)))[0]) == 5 == oracle.sample_greedy(y)
    for bad in (np.nan, np.inf):
        z = x.copy()
        z[1234] = bad
        assert int(host(ikv.argmax(workspace=ws, logits=dev_t(z, dev)))[0]) == -1 == oracle.sample_greedy(z)
    ninf = np.full(1000, -np.inf, np.float32)
    assert int(host(ikv.argmax(workspace=ws, logits=dev_t(ninf, dev)))[0]) == -1
    # unaligned start (scalar path) and a short odd length
    big = dev_t(np.concatenate([[0.0], y]).astype(np.float32), dev)
    assert int(host(ikv.argmax(workspace=ws, logits=big[1:]))[0]) == 5
    w = synth.normal(19, (7,))
    assert int(host(ikv.argmax(workspace=ws, logits=dev_t(w, dev)))[0]) == int(np.argmax(w))
    # the maximum in the last batch of loads, in the scalar tail, at index 0;
    # ties across load batches; and the mirror output
    for n, at in ((151936, 151930), (151937, 151936), (40003, 0), (32768 * 4 + 5, 32768 * 4 - 1)):
        v = synth.normal(20 + n, (n,))
        v[at] = 50.0
        mirror = torch.full((1,), -7, dtype=torch.int32, device=dev)
        tok = ikv.argmax(workspace=ws, logits=dev_t(v, dev), mirror=mirror)
        assert int(host(tok)[0]) == at == int(host(mirror)[0]) == oracle.sample_greedy(v)
    t = synth.normal(21, (100000,))
    t[[8191 * 4 + 1, 8192 * 4 + 2, 99999]] = 40.0       # tie between two load batches
    assert int(host(ikv.argmax(workspace=ws, logits=dev_t(t, dev)))[0]) == 8191 * 4 + 1 == oracle.sample_greedy(t)
    if ws is not None:
        # the workspace form's slices: 151936 logits = 37984 float4 over 64
        # workgroups of 594 float4 (2376 logits); a tie across the first
        # boundary, NaN in the last workgroup's tail, one logit, an all-equal row
        u = synth.normal(22, (151936,))
        u[[2375, 2376]] = 60.0
        assert int(host(ikv.argmax(workspace=ws, logits=dev_t(u, dev)))[0]) == 2375
        u[[2375]] = 0.0
        assert int(host(ikv.argmax(workspace=ws, logits=dev_t(u, dev)))[0]) == 2376
        tail = synth.normal(23, (151939,))
        tail[151938] = np.nan
        assert int(host(ikv.argmax(workspace=ws, logits=dev_t(tail, dev)))[0]) == -1
        one = np.array([3.0], np.float32)
        assert int(host(ikv.argmax(workspace=ws, logits=dev_t(one, dev)))[0]) == 0
        flat = np.full(70000, 2.5, np.float32)
        assert int(host(ikv.argmax(workspace=ws, logits=dev_t(flat, dev)))[0]) == 0
        assert not host(ws)[:4].any()  # the arrival counter is back at zero
    del torch


# ---------------------------------------------------------------------------
# the whole model
# ---------------------------------------------------------------------------

SMALL = qwen3.Qwen3Config(n_layer=4, n_vocab=8192, n_ctx_train=4096)


# |engine - oracle| <= LOGIT_ATOL + LOGIT_RTOL * |oracle| for whole-model
# logits: the same F32 arithmetic summed in other orders through every layer
LOGIT_ATOL, LOGIT_RTOL = 1e-3, 1e-3


def assert_logits_close(got, want, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    print(f"{what}: max |diff| {err.max():.3e}, max |logit| {np.abs(want).max():.3f}", flush=True)
    assert np.all(err <= LOGIT_ATOL + LOGIT_RTOL * np.abs(want)), \
        f"{what}: max |diff| {err.max():.3e} over the bound"


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
    # a decode step took every fusion: per layer attn_norm + q/k/v with the
    # qk-norm + RoPE + append + decode folded in (a short context), o_proj +
    # residual, ffn_norm + SwiGLU, down + residual: 4 launches per layer
    L = SMALL.n_layer
    assert stats["fused_rope_decode"] == L and stats["fused_append_decode"] == L
    assert stats["fused_qkv"] == L and stats["fused_swiglu"] == L and stats["fused_residual"] == 2 * L
    assert stats["fused_norm_mm"] == 2 * L and stats["fused_norm_rope"] == 0
    assert stats["fused_qkv_decode"] == L
    assert stats["launches"] == 4 * L + 3  # + embedding, final norm, logits
    assert t.ttft_s > 0 and t.tpot_s > 0
    # unfused graph (every node its own kernel) gives the same tokens
    eng.set_fusion(False)
    assert eng.generate(prompt, 48)[0] == ref
    eng.close()


def test_decode_steps_replay_a_captured_graph(dev):
    """Decode steps replayed from a captured HIP graph give the tokens of the
    eager steps, across the captures the decode's split plan forces: a
    100-token prompt and 300 tokens are contexts 101..399, captured at 101
    (one split, the decode folded into the q/k/v launch, to 128), 129
    (64-key splits, to 384) and 385."""
    cfg = qwen3.Qwen3Config(n_layer=2, n_vocab=4096, n_ctx_train=4096)
    w = qwen3.synthetic_weights(cfg, synth.config_seed(0, 70), std=0.05)
    prompt = synth.uniform_ints(synth.config_seed(0, 71), 100, cfg.n_vocab)
    eng = engine_with(cfg, w, 400)
    toks, t = eng.generate(prompt, 300)
    st = eng.last_stats()
    assert st["step_replays"] == 299 and st["step_captures"] == 3
    assert t.tpot_s > 0
    eng.set_step_replay(False)
    eager, _ = eng.generate(prompt, 300)
    assert eng.last_stats()["step_replays"] == 0
    assert toks == eager
    # a second sequence on the same engine captures afresh (the graph holds
    # the first sequence's cache rows)
    eng.set_step_replay(True)
    assert eng.generate(prompt, 40)[0] == eager[:40]
    assert eng.last_stats()["step_captures"] == 2
    eng.close()


def test_prefill_appends_are_written_by_their_producers(dev, oracle_pool):
    """A prefill step writes its K rows from the qk-norm + RoPE launch and its
    V rows from the v projection straight into the cache: no copy launches,
    and the tokens (which read those rows back in every later step) stay the
    oracle's, for a skinny-GEMM prompt (20 tokens) and a library-GEMM one (70)."""
    cfg = qwen3.Qwen3Config(n_layer=2, n_vocab=4096, n_ctx_train=4096)
    w = qwen3.synthetic_weights(cfg, synth.config_seed(0, 60), std=0.05)
    for P in (20, 70):
        prompt = synth.uniform_ints(synth.config_seed(0, 61 + P), P, cfg.n_vocab)
        eng = engine_with(cfg, w, P + 16)
        eng.generate(prompt, 1)  # the prefill step alone
        st = eng.last_stats()
        assert st["fused_append"] == 2 * cfg.n_layer
        assert eng.generate(prompt, 16)[0] == oracle.Qwen3Oracle(cfg, w, P + 16).generate(prompt, 16)
        eng.close()


@pytest.mark.parametrize("n_head,n_head_kv,prompt_len,n_gen", [(32, 8, 70, 64), (8, 8, 20, 40)])
def test_other_group_sizes_greedy_tokens_match_oracle(dev, oracle_pool, n_head, n_head_kv,
                                                      prompt_len, n_gen):
    # G = 4 (the Qwen3-8B grouping) with a 70-token prompt: the prefill
    # projections take the library GEMM (m > 64) and decode crosses 128
    # cached tokens into the split-and-merge path; G = 1 with a 20-token
    # prompt takes the few-token MFMA projections.
    cfg = qwen3.Qwen3Config(n_layer=2, n_head=n_head, n_head_kv=n_head_kv, n_vocab=4096,
                            n_ctx_train=4096)
    # std 0.05 rather than the benchmarks' 0.02: with two layers the larger
    # weights make attention and the MLP move the argmax, so the tokens vary
    w = qwen3.synthetic_weights(cfg, synth.config_seed(0, 40 + n_head), std=0.05)
    prompt = synth.uniform_ints(synth.config_seed(0, 41 + n_head), prompt_len, cfg.n_vocab)
    ref = oracle.Qwen3Oracle(cfg, w, prompt_len + n_gen).generate(prompt, n_gen)
    eng = engine_with(cfg, w, prompt_len + n_gen)
    assert eng.generate(prompt, n_gen)[0] == ref
    eng.set_fusion(False)
    assert eng.generate(prompt, n_gen)[0] == ref
    eng.close()


def test_untied_gguf_model_uses_its_output_projection(dev, oracle_pool, tmp_path):
    # a GGUF file with output.weight (src/model.cpp:203-210) loads untied and
    # its logits come from that projection: the tokens equal the oracle's
    # with output.weight, and differ from those of the tied embedding
    from ikv import gguf
    cfg = qwen3.Qwen3Config(n_layer=2, n_vocab=4096, n_ctx_train=4096, untied_output=1)
    path = tmp_path / "untied.gguf"
    gguf.write_qwen3_synthetic(path, cfg, seed=synth.config_seed(0, 50), std=0.05, threads=8)
    w = qwen3.synthetic_weights(cfg, synth.config_seed(0, 50), std=0.05)
    prompt = synth.uniform_ints(synth.config_seed(0, 51), 24, cfg.n_vocab)
    ref = oracle.Qwen3Oracle(cfg, w, 64).generate(prompt, 32)
    tied = {k: v for k, v in w.items() if k != "output.weight"}
    ref_tied = oracle.Qwen3Oracle(cfg, tied, 64).generate(prompt, 32)
    assert ref != ref_tied
    eng = gguf.load_qwen3(path, 64)
    assert eng.cfg.untied_output == 1 and eng.tensor_names()[-1] == "output.weight"
    assert eng.generate(prompt, 32)[0] == ref
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
    steps = [0, 1, 64, 127]  # the prefill's row, the first decode, mid-run, last
    eng.capture_logits(steps)
    toks, _ = eng.generate(prompt, 128)
    got = eng.captured_logits()
    eng.close()
    orc = oracle.Qwen3Oracle(cfg, w, 160)
    ref = orc.generate(prompt, 128, keep_logits=steps)
    assert toks == ref
    # logits at those steps: every one of the 151936 within the model-level
    # bound (F32 sums in another order through 28 layers)
    for k, st in enumerate(steps):
        assert_logits_close(got[k], orc.kept[st], f"config 0 step {st}")


# ---------------------------------------------------------------------------
# folded forms equal the separate ops bit for bit
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("k", [1024, 4096])
def test_norm_folded_into_gemv_equals_separate_norm(dev, k):
    x = synth.normal(20 + k, (k,)) * 2
    nw = 1 + 0.2 * synth.normal(21, (k,))
    ws = [synth.normal(22 + i, (n, k), 0.02) for i, n in enumerate((512, 256, 256))]
    xd, nwd = dev_t(x, dev), dev_t(nw, dev)
    normed = ikv.rms_norm(xd[None], nwd, 1e-6)[0]
    sep = [host(o) for o in ikv.gemv3(*[dev_t(w, dev) for w in ws], normed)]
    fused = [host(o) for o in ikv.gemv3(*[dev_t(w, dev) for w in ws], xd, norm_w=nwd, eps=1e-6)]
    for a, b in zip(sep, fused):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    wg, wu = dev_t(ws[1], dev), dev_t(ws[2], dev)
    sep = host(ikv.gemv_swiglu(wg, wu, normed))
    fused = host(ikv.gemv_swiglu(wg, wu, xd, norm_w=nwd, eps=1e-6))
    assert np.array_equal(sep.view(np.uint32), fused.view(np.uint32))
    # and the model-width norm itself matches the reference's float result on these rows
    ref = oracle.rms_norm(x[None], nw, 1e-6)[0]
    assert np.array_equal(host(normed).view(np.uint32), ref.view(np.uint32))


# Products of at least 16M weight floats stage their input in LDS once per
# workgroup and walk several row groups per wave: q/k/v at Qwen3-8B width
# (one group per wave), twice as many rows (two per wave), odd row counts
# (one row per group), and the 8B SwiGLU pair (four rows per wave).
@pytest.mark.parametrize("ns", [(4096, 1024, 1024), (8192, 2048, 2048), (4095, 1025, 1023)])
def test_staged_gemv3_folded_equals_separate_norm(dev, oracle_pool, ns):
    k = 4096
    x = synth.normal(30, (k,)) * 2
    nw = 1 + 0.2 * synth.normal(31, (k,))
    ws = [synth.normal(32 + i, (n, k), 0.02) for i, n in enumerate(ns)]
    wd = [dev_t(w, dev) for w in ws]
    xd, nwd = dev_t(x, dev), dev_t(nw, dev)
    normed = ikv.rms_norm(xd[None], nwd, 1e-6)[0]
    sep = [host(o) for o in ikv.gemv3(*wd, normed)]
    fused = [host(o) for o in ikv.gemv3(*wd, xd, norm_w=nwd, eps=1e-6)]
    xn = host(normed)
    for w, a, b in zip(ws, sep, fused):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert proj_close(a, w, xn[None], oracle.mul_mat(w, xn))


def test_staged_swiglu_folded_equals_separate_norm(dev):
    n_out, k = 12288, 4096
    x = synth.normal(40, (k,)) * 2
    nw = 1 + 0.2 * synth.normal(41, (k,))
    wg = dev_t(synth.normal(42, (n_out, k), 0.02), dev)
    wu = dev_t(synth.normal(43, (n_out, k), 0.02), dev)
    xd, nwd = dev_t(x, dev), dev_t(nw, dev)
    normed = ikv.rms_norm(xd[None], nwd, 1e-6)[0]
    sep = host(ikv.gemv_swiglu(wg, wu, normed))
    fused = host(ikv.gemv_swiglu(wg, wu, xd, norm_w=nwd, eps=1e-6))
    assert np.array_equal(sep.view(np.uint32), fused.view(np.uint32))


@pytest.mark.parametrize("Hq,Hkv,ctx,near", [(16, 8, 0, False), (16, 8, 37, False),
                                             (16, 8, 4096, False), (32, 8, 1000, False),
                                             (8, 8, 300, False), (64, 8, 129, False),
                                             (16, 8, 37, True), (32, 8, 1000, True)])
def test_decode_with_qk_rope_equals_separate_ops(dev, oracle_pool, Hq, Hkv, ctx, near):
    """near: q and k rows whose norm scales sit closest to float rounding
    midpoints, so that the folded prologue's certified sum falls back to the
    index-order one."""
    import torch
    D = 128
    th = oracle.rope_theta_table(1e6, D, 8192)
    s, c = ikv.rope_sincos_table(th)
    sd, cd = dev_t(s, dev), dev_t(c, dev)
    qn_w = 1 + 0.3 * synth.normal(30, (D,))
    kn_w = 1 + 0.3 * synth.normal(31, (D,))
    q_raw = synth.normal(32 + ctx, (Hq, D)) * 2
    k_raw = synth.normal(33 + ctx, (Hkv, D)) * 2
    if near:
        from test_gpu_kernels import near_midpoint_rows
        rows, _ = near_midpoint_rows(D, 1 << 20, 777 + ctx, Hq + Hkv)
        q_raw, k_raw = rows[:Hq].copy(), rows[Hq:].copy()
    v_new = synth.normal(34 + ctx, (Hkv, D))
    hist_k = synth.normal(35 + ctx, (ctx + 1, Hkv, D))
    hist_v = synth.normal(36 + ctx, (ctx + 1, Hkv, D))
    pos = torch.tensor([ctx], dtype=torch.int32, device=dev)
    # separate: qk-norm+rope, then decode with fused append
    q_rot = ikv.qk_norm_rope(dev_t(q_raw[None], dev), dev_t(qn_w, dev), pos, 1e-6, sd, cd)[0]
    k_rot = ikv.qk_norm_rope(dev_t(k_raw[None], dev), dev_t(kn_w, dev), pos, 1e-6, sd, cd)[0]
    kc1, vc1 = dev_t(hist_k, dev), dev_t(hist_v, dev)
    out1 = ikv.attn_decode(q_rot, kc1, vc1, ctx + 1, k_new=k_rot, v_new=dev_t(v_new, dev))
    # folded
    kc2, vc2 = dev_t(hist_k, dev), dev_t(hist_v, dev)
    out2 = ikv.attn_decode_rope(dev_t(q_raw, dev), dev_t(k_raw, dev), dev_t(v_new, dev), kc2, vc2,
                                ctx + 1, dev_t(qn_w, dev), dev_t(kn_w, dev), 1e-6, pos, sd, cd)
    assert np.array_equal(host(kc1).view(np.uint32), host(kc2).view(np.uint32))
    assert np.array_equal(host(vc1).view(np.uint32), host(vc2).view(np.uint32))
    assert np.array_equal(host(out1).view(np.uint32), host(out2).view(np.uint32))
    # and against the oracle chain
    qo = oracle.rope_neox(oracle.rms_norm(q_raw[None], qn_w, 1e-6), np.array([ctx], np.int32), th)[0]
    ko = oracle.rope_neox(oracle.rms_norm(k_raw[None], kn_w, 1e-6), np.array([ctx], np.int32), th)[0]
    hk, hv = hist_k.copy(), hist_v.copy()
    want = oracle.decode_append_attn(qo, ko, v_new, hk, hv, ctx)
    assert np.array_equal(host(kc2).view(np.uint32), hk.view(np.uint32))
    got = host(out2).astype(np.float64)
    assert np.all(np.abs(got - want) <= 1e-5 + 1e-4 * np.abs(want))


@pytest.mark.parametrize("Hq,Hkv,K,n_kv,norm", [(16, 8, 1024, 1, True), (16, 8, 1024, 33, True),
                                               (16, 8, 1024, 64, True), (16, 8, 1024, 65, False),
                                               (16, 8, 1024, 128, True), (32, 8, 2048, 100, True),
                                               (8, 8, 1024, 77, True), (64, 8, 1024, 50, True)])
def test_qkv_attn_folded_equals_separate_launches(dev, oracle_pool, Hq, Hkv, K, n_kv, norm):
    """ikv_qkv_attn_decode_f32 (q/k/v projection with the short-context decode
    folded in) against ikv_gemv3_f32 followed by ikv_attn_decode_rope_f32:
    the projections, the output and both caches bit for bit, twice in a row
    (the arrival counters must come back to zero)."""
    import torch
    D = 128
    th = oracle.rope_theta_table(1e6, D, 4096)
    s, c = ikv.rope_sincos_table(th)
    sd, cd = dev_t(s, dev), dev_t(c, dev)
    seed = 600 + Hq + n_kv + K
    wq = dev_t(synth.normal(seed, (Hq * D, K), 0.02), dev)
    wk = dev_t(synth.normal(seed + 1, (Hkv * D, K), 0.02), dev)
    wv = dev_t(synth.normal(seed + 2, (Hkv * D, K), 0.02), dev)
    x = dev_t(synth.normal(seed + 3, (K,)), dev)
    an = dev_t(1 + 0.2 * synth.normal(seed + 4, (K,)), dev) if norm else None
    qn_w = dev_t(1 + 0.3 * synth.normal(seed + 5, (D,)), dev)
    kn_w = dev_t(1 + 0.3 * synth.normal(seed + 6, (D,)), dev)
    hist_k = synth.normal(seed + 7, (n_kv, Hkv, D))
    hist_v = synth.normal(seed + 8, (n_kv, Hkv, D))
    pos = torch.tensor([n_kv - 1], dtype=torch.int32, device=dev)
    ws = ikv.decode_workspace(Hq, Hkv, D, n_kv, device=dev)
    for rep in range(2):
        q, k, v = ikv.gemv3(wq, wk, wv, x, norm_w=an, eps=1e-6)
        kc1, vc1 = dev_t(hist_k, dev), dev_t(hist_v, dev)
        out1 = ikv.attn_decode_rope(q.view(Hq, D), k.view(Hkv, D), v.view(Hkv, D), kc1, vc1, n_kv,
                                    qn_w, kn_w, 1e-6, pos, sd, cd, workspace=ws)
        kc2, vc2 = dev_t(hist_k, dev), dev_t(hist_v, dev)
        out2, q2, k2, v2 = ikv.qkv_attn_decode(wq, wk, wv, x, kc2, vc2, n_kv, qn_w, kn_w, 1e-6, pos,
                                               sd, cd, attn_norm_w=an, attn_eps=1e-6, workspace=ws)
        for a, b, what in ((q, q2, "q"), (k, k2, "k"), (v, v2, "v"), (out1, out2, "out"),
                           (kc1, kc2, "K cache"), (vc1, vc2, "V cache")):
            assert np.array_equal(host(a).reshape(-1).view(np.uint32),
                                  host(b).reshape(-1).view(np.uint32)), f"rep {rep}: {what}"
    assert not host(ws)[:Hkv * 64].any()  # every arrival counter back at zero


@pytest.mark.parametrize("Hq,n_kv", [(16, 1), (16, 41), (16, 64), (16, 100), (16, 128), (32, 77),
                                     (16, 129), (16, 4097), (32, 4097)])
def test_decode_ignores_the_unwritten_rows(dev, Hq, n_kv):
    """Every one-token decode form reads only cache rows [0, n_kv-1) and the
    new row it is given: the new row's cache slot and the rows past it are not
    written yet, and an allocation may hand them over holding NaN or inf. A
    lane whose row lies past the context still multiplies a V row by a zero
    weight, so such rows must come from the new token, not from that slot.
    Outputs with the slot and the rows past it set to NaN / inf equal, bit for
    bit, those with finite values there."""
    import torch
    Hkv, D, K, cap = 8, 128, 1024, n_kv + 70
    th = oracle.rope_theta_table(1e6, D, cap + 8)
    s, c = ikv.rope_sincos_table(th)
    sd, cd = dev_t(s, dev), dev_t(c, dev)
    seed = 1300 + n_kv + Hq
    qn_w = dev_t(1 + 0.3 * synth.normal(seed, (D,)), dev)
    kn_w = dev_t(1 + 0.3 * synth.normal(seed + 1, (D,)), dev)
    hist_k = synth.normal(seed + 2, (cap, Hkv, D))
    hist_v = synth.normal(seed + 3, (cap, Hkv, D))
    q = dev_t(synth.normal(seed + 4, (Hq, D)), dev)
    k_new = dev_t(synth.normal(seed + 5, (Hkv, D)), dev)
    v_new = dev_t(synth.normal(seed + 6, (Hkv, D)), dev)
    pos = torch.tensor([n_kv - 1], dtype=torch.int32, device=dev)
    ws = ikv.decode_workspace(Hq, Hkv, D, n_kv, device=dev)
    fold = n_kv <= 128
    if fold:
        wq = dev_t(synth.normal(seed + 7, (Hq * D, K), 0.02), dev)
        wk = dev_t(synth.normal(seed + 8, (Hkv * D, K), 0.02), dev)
        wv = dev_t(synth.normal(seed + 9, (Hkv * D, K), 0.02), dev)
        x = dev_t(synth.normal(seed + 10, (K,)), dev)

    def run(fill):
        kk, vv = hist_k.copy(), hist_v.copy()
        if fill is not None:
            kk[n_kv - 1:] = fill
            vv[n_kv - 1:] = fill
        outs = []
        for form in ("plain", "rope", "fold"):
            if form == "fold" and not fold:
                continue
            kc, vc = dev_t(kk, dev), dev_t(vv, dev)
            if form == "plain":
                o = ikv.attn_decode(q, kc, vc, n_kv, k_new=k_new, v_new=v_new, workspace=ws)
            elif form == "rope":
                o = ikv.attn_decode_rope(q, k_new, v_new, kc, vc, n_kv, qn_w, kn_w, 1e-6, pos, sd, cd,
                                         workspace=ws)
            else:
                o, *_ = ikv.qkv_attn_decode(wq, wk, wv, x, kc, vc, n_kv, qn_w, kn_w, 1e-6, pos, sd, cd,
                                            workspace=ws)
            outs.append((form, host(o).copy(), host(kc)[:n_kv].copy(), host(vc)[:n_kv].copy()))
        return outs

    base = run(None)
    for fill in (np.nan, np.inf, -np.inf):
        for (form, o0, k0, v0), (_, o1, k1, v1) in zip(base, run(fill)):
            assert np.isfinite(o1).all(), f"{form}, slot {fill}: non-finite output"
            for a, b, what in ((o0, o1, "out"), (k0, k1, "K rows"), (v0, v1, "V rows")):
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{form}, slot {fill}: {what}"


@pytest.mark.parametrize("Hq,n_kv_lo,width", [(16, 33, 256), (16, 129, 256), (16, 2050, 256),
                                               (16, 2113, 128), (32, 300, 200)])
def test_decode_replay_equals_per_context_launches(dev, Hq, n_kv_lo, width):
    """The replay forms (context read from pos on the device, launch planned
    for the replay limit) against the per-context launches at contexts
    across the limit's range: outputs and appended cache rows bit for bit.
    One replay launch object is reused, as a captured graph would be."""
    import torch
    Hkv, D, K = 8, 128, 1024
    m = ikv.decode_replay_limit(Hq, Hkv, D, n_kv_lo, width)
    assert n_kv_lo <= m < n_kv_lo + width
    th = oracle.rope_theta_table(1e6, D, m + 8)
    s, c = ikv.rope_sincos_table(th)
    sd, cd = dev_t(s, dev), dev_t(c, dev)
    seed = 900 + n_kv_lo + Hq
    qn_w = dev_t(1 + 0.3 * synth.normal(seed, (D,)), dev)
    kn_w = dev_t(1 + 0.3 * synth.normal(seed + 1, (D,)), dev)
    hist_k = synth.normal(seed + 2, (m, Hkv, D))
    hist_v = synth.normal(seed + 3, (m, Hkv, D))
    ws_r = ikv.decode_workspace(Hq, Hkv, D, m, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    fold = m <= 128  # the q/k/v launch takes the decode in
    if fold:
        wq = dev_t(synth.normal(seed + 4, (Hq * D, K), 0.02), dev)
        wk = dev_t(synth.normal(seed + 5, (Hkv * D, K), 0.02), dev)
        wv = dev_t(synth.normal(seed + 6, (Hkv * D, K), 0.02), dev)
        an = dev_t(1 + 0.2 * synth.normal(seed + 7, (K,)), dev)
    for n_kv in sorted({n_kv_lo, (n_kv_lo + m) // 2, m}):
        pos.fill_(n_kv - 1)
        g = seed + 10 * n_kv
        kc1, vc1 = dev_t(hist_k, dev), dev_t(hist_v, dev)
        kc2, vc2 = dev_t(hist_k, dev), dev_t(hist_v, dev)
        ws1 = ikv.decode_workspace(Hq, Hkv, D, n_kv, device=dev)
        if fold:
            x = dev_t(synth.normal(g, (K,)), dev)
            out1, *_ = ikv.qkv_attn_decode(wq, wk, wv, x, kc1, vc1, n_kv, qn_w, kn_w, 1e-6, pos, sd,
                                           cd, attn_norm_w=an, attn_eps=1e-6, workspace=ws1)
            out2, *_ = ikv.qkv_attn_decode(wq, wk, wv, x, kc2, vc2, m, qn_w, kn_w, 1e-6, pos, sd,
                                           cd, attn_norm_w=an, attn_eps=1e-6, workspace=ws_r,
                                           replay=True)
        else:
            q_raw = dev_t(synth.normal(g, (Hq, D)), dev)
            k_raw = dev_t(synth.normal(g + 1, (Hkv, D)), dev)
            v_new = dev_t(synth.normal(g + 2, (Hkv, D)), dev)
            out1 = ikv.attn_decode_rope(q_raw, k_raw, v_new, kc1, vc1, n_kv, qn_w, kn_w, 1e-6, pos,
                                        sd, cd, workspace=ws1)
            out2 = ikv.attn_decode_rope(q_raw, k_raw, v_new, kc2, vc2, m, qn_w, kn_w, 1e-6, pos,
                                        sd, cd, workspace=ws_r, replay=True)
        for a, b, what in ((out1, out2, "out"), (kc1, kc2, "K cache"), (vc1, vc2, "V cache")):
            assert np.array_equal(host(a).reshape(-1).view(np.uint32),
                                  host(b).reshape(-1).view(np.uint32)), f"n_kv {n_kv}: {what}"


@pytest.mark.parametrize("Hq,n_kv_lo,width,bt", [(16, 2050, 256, 256), (16, 300, 200, 64),
                                                  (32, 129, 256, 128), (16, 40, 256, 64)])
def test_paged_decode_replay_equals_contiguous_launches(dev, Hq, n_kv_lo, width, bt):
    """The paged replay form (context from pos, planned for the replay
    limit) over a shuffled pool whose block table holds entries only for the
    blocks of keys [0, n_kv) (later entries -1, as before a sequence grows
    into them) against the contiguous per-context launch: outputs and the
    appended rows bit for bit, and no block-table error raised."""
    import torch
    Hkv, D = 8, 128
    m = ikv.decode_replay_limit(Hq, Hkv, D, n_kv_lo, width)
    th = oracle.rope_theta_table(1e6, D, m + 8)
    s, c = ikv.rope_sincos_table(th)
    sd, cd = dev_t(s, dev), dev_t(c, dev)
    seed = 1900 + n_kv_lo + Hq + bt
    qn_w = dev_t(1 + 0.3 * synth.normal(seed, (D,)), dev)
    kn_w = dev_t(1 + 0.3 * synth.normal(seed + 1, (D,)), dev)
    hist_k = synth.normal(seed + 2, (m, Hkv, D))
    hist_v = synth.normal(seed + 3, (m, Hkv, D))
    n_blocks = -(-m // bt)
    pool_blocks = n_blocks + 3
    order = np.random.default_rng(seed).permutation(pool_blocks)[:n_blocks].astype(np.int32)
    ws_r = ikv.decode_workspace(Hq, Hkv, D, m, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    for n_kv in sorted({n_kv_lo, (n_kv_lo + m) // 2, m}):
        pos.fill_(n_kv - 1)
        g = seed + 10 * n_kv
        kc1, vc1 = dev_t(hist_k, dev), dev_t(hist_v, dev)
        pools = []
        for hist in (hist_k, hist_v):
            pool = np.zeros((pool_blocks * bt, Hkv, D), np.float32)
            for b, blk in enumerate(order):
                rows = hist[b * bt:(b + 1) * bt]
                pool[blk * bt:blk * bt + len(rows)] = rows
            pools.append(dev_t(pool, dev))
        live = -(-n_kv // bt)  # blocks holding keys [0, n_kv)
        table = torch.tensor(np.where(np.arange(n_blocks) < live, order, -1).astype(np.int32),
                             device=dev)
        page_status = torch.zeros(1, dtype=torch.int32, device=dev)
        ws1 = ikv.decode_workspace(Hq, Hkv, D, n_kv, device=dev)
        q_raw = dev_t(synth.normal(g, (Hq, D)), dev)
        k_raw = dev_t(synth.normal(g + 1, (Hkv, D)), dev)
        v_new = dev_t(synth.normal(g + 2, (Hkv, D)), dev)
        out1 = ikv.attn_decode_rope(q_raw, k_raw, v_new, kc1, vc1, n_kv, qn_w, kn_w, 1e-6, pos,
                                    sd, cd, workspace=ws1)
        out2 = ikv.attn_decode_rope_paged(q_raw, k_raw, v_new, pools[0], pools[1], table, bt, m,
                                          qn_w, kn_w, 1e-6, pos, sd, cd, page_status=page_status,
                                          workspace=ws_r, replay=True)
        assert np.array_equal(host(out1).view(np.uint32), host(out2).view(np.uint32)), n_kv
        assert int(host(page_status)[0]) == 0, f"n_kv {n_kv}: block-table error raised"
        t = n_kv - 1
        row = order[t // bt] * bt + t % bt
        for cont, pool in ((kc1, pools[0]), (vc1, pools[1])):
            assert np.array_equal(host(cont)[t].view(np.uint32), host(pool)[row].view(np.uint32))


def test_decode_replay_position_past_plan_is_flagged(dev):
    import torch
    Hq, Hkv, D = 16, 8, 128
    th = oracle.rope_theta_table(1e6, D, 1024)
    s, c = ikv.rope_sincos_table(th)
    sd, cd = dev_t(s, dev), dev_t(c, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(17)
    kc = torch.zeros((400, Hkv, D), device=dev)
    vc = torch.zeros_like(kc)
    kc[:384] = torch.randn((384, Hkv, D), generator=g, device=dev)  # committed history
    vc[:384] = torch.randn((384, Hkv, D), generator=g, device=dev)
    k0, v0 = kc.clone(), vc.clone()
    t = torch.ones((Hq, D), device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    pos = torch.tensor([384], dtype=torch.int32, device=dev)  # context 385 > planned 384
    ikv.attn_decode_rope(t, t[:Hkv], t[:Hkv], kc, vc, 384, t[0], t[0], 1e-6, pos, sd, cd,
                         status=status, replay=True)
    torch.cuda.synchronize()
    assert int(status.item()) & ikv.STATUS_POSITION
    # no append: the committed rows (the last planned one included) keep their
    # bits, and nothing is written past the planned rows
    assert torch.equal(kc.view(torch.int32), k0.view(torch.int32))
    assert torch.equal(vc.view(torch.int32), v0.view(torch.int32))


def test_qkv_decode_replay_position_past_plan_appends_nothing(dev):
    # the same for the q/k/v-folded replay form (planned for 128 keys)
    import torch
    Hq, Hkv, D, K = 16, 8, 128, 1024
    th = oracle.rope_theta_table(1e6, D, 1024)
    s, c = ikv.rope_sincos_table(th)
    sd, cd = dev_t(s, dev), dev_t(c, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(18)
    w = lambda n: torch.randn((n, K), generator=g, device=dev) * 0.02  # noqa: E731
    x = torch.randn(K, generator=g, device=dev)
    kc = torch.randn((160, Hkv, D), generator=g, device=dev)
    vc = torch.randn((160, Hkv, D), generator=g, device=dev)
    k0, v0 = kc.clone(), vc.clone()
    ones = torch.ones(D, device=dev)
    for p in (128, 150, -1):
        status = torch.zeros(1, dtype=torch.int32, device=dev)
        pos = torch.tensor([p], dtype=torch.int32, device=dev)
        ikv.qkv_attn_decode(w(Hq * D), w(Hkv * D), w(Hkv * D), x, kc, vc, 128, ones, ones, 1e-6,
                            pos, sd, cd, status=status, replay=True)
        torch.cuda.synchronize()
        assert int(status.item()) & ikv.STATUS_POSITION, p
        assert torch.equal(kc.view(torch.int32), k0.view(torch.int32)), p
        assert torch.equal(vc.view(torch.int32), v0.view(torch.int32)), p


def test_qkv_attn_rejects_long_contexts(dev):
    import torch
    D = 128
    t = torch.zeros(1 << 20, device=dev)
    with pytest.raises(ikv.IkvError) as e:
        ikv.qkv_attn_decode(t.view(-1, 1024)[:2048], t.view(-1, 1024)[:1024], t.view(-1, 1024)[:1024],
                            t[:1024], t.view(-1, 8, D)[:200], t.view(-1, 8, D)[:200], 129, t[:D],
                            t[:D], 1e-6, torch.zeros(1, dtype=torch.int32, device=dev),
                            t.view(-1, 64)[:10], t.view(-1, 64)[:10])
    assert e.value.rc == -errno.ENOTSUP


def test_decode_with_qk_rope_bad_position_is_flagged(dev):
    import torch
    D = 128
    th = oracle.rope_theta_table(1e6, D, 64)
    s, c = ikv.rope_sincos_table(th)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    kc = torch.zeros((11, 8, D), device=dev)
    vc = torch.zeros((11, 8, D), device=dev)
    pos = torch.tensor([64], dtype=torch.int32, device=dev)     # outside the 64-row table
    ones = torch.ones(D, device=dev)
    ikv.attn_decode_rope(torch.ones((16, D), device=dev), torch.ones((8, D), device=dev),
                         torch.ones((8, D), device=dev), kc, vc, 11, ones, ones, 1e-6, pos,
                         dev_t(s, dev), dev_t(c, dev), status=status)
    assert int(host(status)[0]) == ikv.STATUS_POSITION
    assert not host(kc)[10].any()       # the appended key row is zeros, not garbage


def test_engine_from_gguf_file_equals_synthetic_init(dev, tmp_path):
    from ikv import gguf
    cfg = qwen3.Qwen3Config(n_layer=2, n_vocab=4096, n_ctx_train=4096)
    path = tmp_path / "small.gguf"
    gguf.write_qwen3_synthetic(path, cfg, seed=0xABC, threads=4)
    prompt = synth.uniform_ints(5, 24, cfg.n_vocab)
    a = gguf.load_qwen3(path, 128)
    b = qwen3.Qwen3Engine(cfg, 128)
    b.init_synthetic(0xABC)
    assert a.generate(prompt, 20)[0] == b.generate(prompt, 20)[0]
    a.close()
    b.close()
