"""Paged KV cache on the GPU: the block-table forms of append, decode,
decode with qk-norm + RoPE, and prefill.

A paged pool holds the same logical cache as a contiguous one, with each
block of block_tokens rows moved to the pool row the block table names. The
kernels walk the same splits and tiles with the same arithmetic, so every
result must be bit-identical to the contiguous entry point's on the same
logical cache (and, through those, within the attention tolerance of the
oracle, which one case re-checks directly).
"""
import numpy as np
import pytest
import torch

import ikv
import oracle
from ikv import synth

pytestmark = pytest.mark.gpu

D = 128


def bits(t):
    a = t.cpu().numpy() if hasattr(t, "cpu") else np.asarray(t)
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def gen(seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


def rand(g, shape):
    return torch.randn(shape, generator=g, device="cuda", dtype=torch.float32)


def paged_copy(cache, bt, n_pool_blocks, seed, fill=-777.0):
    """Pool [n_pool_blocks * bt, H, D] holding `cache`'s rows block by block at
    the blocks of a random table; every other pool row is `fill`."""
    n_blocks = (cache.shape[0] + bt - 1) // bt
    rng = np.random.default_rng(seed)
    table = rng.permutation(n_pool_blocks)[:n_blocks].astype(np.int32)
    pool = torch.full((n_pool_blocks * bt,) + tuple(cache.shape[1:]), fill, device="cuda")
    for b, blk in enumerate(table):
        n = min(bt, cache.shape[0] - b * bt)
        pool[blk * bt:blk * bt + n] = cache[b * bt:b * bt + n]
    return pool, torch.tensor(table, device="cuda")


def gather(pool, table, bt, n):
    """Logical rows [0, n) of a paged pool."""
    t = table.cpu().numpy()
    rows = [int(t[i // bt]) * bt + i % bt for i in range(n)]
    return pool[torch.tensor(rows, device="cuda", dtype=torch.long)]


@pytest.mark.parametrize("bt,first,n", [(64, 0, 1), (64, 63, 2), (128, 100, 300), (256, 0, 1024),
                                        (64, 5, 0)])
def test_append_paged_scatters_bit_exact(dev, bt, first, n):
    g = gen(11 + bt + first + n)
    n_pool = (first + n + bt - 1) // bt + 3
    pool = torch.full((n_pool * bt, 8, D), 55.5, device=dev)
    table = torch.tensor(np.random.default_rng(bt + n).permutation(n_pool).astype(np.int32),
                         device=dev)
    src = rand(g, (n, 8, D))
    before = pool.clone()
    ikv.append_paged(pool, src, table, bt, first)
    torch.cuda.synchronize()
    want = before.clone()
    t = table.cpu().numpy()
    for i in range(n):
        r = int(t[(first + i) // bt]) * bt + (first + i) % bt
        want[r] = src[i]
    assert np.array_equal(bits(pool), bits(want))


@pytest.mark.parametrize("Hq,n_kv,bt", [(16, 1, 64), (16, 64, 64), (16, 65, 64), (16, 200, 128),
                                        (16, 4097, 64), (16, 4097, 256), (32, 4352, 128),
                                        (8, 777, 64), (64, 1500, 192), (16, 20000, 512)])
def test_decode_paged_equals_contiguous_bitwise(dev, Hq, n_kv, bt):
    Hkv = 8
    g = gen(21 + Hq + n_kv + bt)
    k = rand(g, (n_kv, Hkv, D))
    v = rand(g, (n_kv, Hkv, D))
    q = rand(g, (Hq, D))
    kn = rand(g, (Hkv, D))
    vn = rand(g, (Hkv, D))
    n_pool = (n_kv + bt - 1) // bt + 5
    kp, table = paged_copy(k, bt, n_pool, seed=n_kv)
    vp, _ = paged_copy(v, bt, n_pool, seed=n_kv)
    out_c = ikv.attn_decode(q, k, v, n_kv, k_new=kn, v_new=vn)
    out_p = ikv.attn_decode_paged(q, kp, vp, table, bt, n_kv, k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out_c), bits(out_p))
    # the fused append landed in the pool row of token n_kv - 1, bit for bit
    assert np.array_equal(bits(gather(kp, table, bt, n_kv)), bits(k))
    assert np.array_equal(bits(gather(vp, table, bt, n_kv)), bits(v))
    # rows of the pool that no block of the table names are untouched
    used = set(int(b) for b in table.cpu().numpy())
    free = [b for b in range(n_pool) if b not in used]
    for b in free[:2]:
        assert torch.all(kp[b * bt:(b + 1) * bt] == -777.0)


def test_decode_paged_matches_oracle(dev, oracle_pool):
    bt, n_kv = 64, 1000
    g = gen(5)
    k = rand(g, (n_kv, 8, D))
    v = rand(g, (n_kv, 8, D))
    q = rand(g, (16, D))
    kp, table = paged_copy(k, bt, 40, seed=9)
    vp, _ = paged_copy(v, bt, 40, seed=9)
    out = ikv.attn_decode_paged(q, kp, vp, table, bt, n_kv).cpu().numpy().astype(np.float64)
    want = oracle.flash_attn(q.cpu().numpy()[None], k.cpu().numpy(), v.cpu().numpy(), n_kv - 1)[0]
    assert np.all(np.abs(out - want) <= 1e-5 + 1e-4 * np.abs(want))


@pytest.mark.parametrize("Hq,ctx,bt", [(16, 0, 64), (16, 63, 64), (16, 4096, 128), (32, 1000, 64)])
def test_decode_rope_paged_equals_contiguous_bitwise(dev, Hq, ctx, bt):
    Hkv = 8
    th = oracle.rope_theta_table(1e6, D, 8192)
    s, c = ikv.rope_sincos_table(th)
    sd, cd = torch.tensor(s, device=dev), torch.tensor(c, device=dev)
    qn_w = torch.tensor(1 + 0.3 * synth.normal(30, (D,)), device=dev)
    kn_w = torch.tensor(1 + 0.3 * synth.normal(31, (D,)), device=dev)
    g = gen(40 + ctx)
    q_raw = rand(g, (Hq, D)) * 2
    k_raw = rand(g, (Hkv, D)) * 2
    v_new = rand(g, (Hkv, D))
    hist_k = rand(g, (ctx + 1, Hkv, D))
    hist_v = rand(g, (ctx + 1, Hkv, D))
    pos = torch.tensor([ctx], dtype=torch.int32, device=dev)
    n_pool = (ctx + 1 + bt - 1) // bt + 2
    kp, table = paged_copy(hist_k, bt, n_pool, seed=ctx + 1)
    vp, _ = paged_copy(hist_v, bt, n_pool, seed=ctx + 1)
    kc, vc = hist_k.clone(), hist_v.clone()
    out_c = ikv.attn_decode_rope(q_raw, k_raw, v_new, kc, vc, ctx + 1, qn_w, kn_w, 1e-6, pos, sd, cd)
    out_p = ikv.attn_decode_rope_paged(q_raw, k_raw, v_new, kp, vp, table, bt, ctx + 1, qn_w, kn_w,
                                       1e-6, pos, sd, cd)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out_c), bits(out_p))
    assert np.array_equal(bits(gather(kp, table, bt, ctx + 1)), bits(kc))
    assert np.array_equal(bits(gather(vp, table, bt, ctx + 1)), bits(vc))


@pytest.mark.parametrize("n_q,n_past,Hq,bt", [(1, 0, 16, 64), (37, 0, 16, 64), (300, 0, 16, 128),
                                              (2048, 0, 16, 256), (17, 100, 16, 64),
                                              (128, 1000, 32, 64), (500, 77, 8, 192)])
def test_prefill_paged_equals_contiguous_bitwise(dev, n_q, n_past, Hq, bt):
    Hkv = 8
    n_kv = n_past + n_q
    g = gen(60 + n_q + n_past + Hq)
    q = rand(g, (n_q, Hq, D))
    k = rand(g, (n_kv, Hkv, D))
    v = rand(g, (n_kv, Hkv, D))
    n_pool = (n_kv + bt - 1) // bt + 3
    kp, table = paged_copy(k, bt, n_pool, seed=n_kv + 3)
    vp, _ = paged_copy(v, bt, n_pool, seed=n_kv + 3)
    out_c = ikv.attn_prefill(q, k, v, n_past)
    out_p = ikv.attn_prefill_paged(q, kp, vp, table, bt, n_past)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out_c), bits(out_p))


def test_bad_block_entry_is_flagged_not_faulted(dev):
    bt, n_kv = 64, 300
    g = gen(77)
    kp = rand(g, (6 * bt, 8, D))
    vp = rand(g, (6 * bt, 8, D))
    q = rand(g, (16, D))
    table = torch.tensor([0, 1, 9, 3, 4], dtype=torch.int32, device=dev)  # 9: outside 6 blocks
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    ikv.attn_decode_paged(q, kp, vp, table, bt, n_kv, status=status)
    torch.cuda.synchronize()
    assert int(status.cpu()[0]) == ikv.STATUS_BLOCK
    status.zero_()
    ikv.attn_prefill_paged(rand(g, (n_kv, 16, D)), kp, vp, table, bt, 0, status=status)
    torch.cuda.synchronize()
    assert int(status.cpu()[0]) == ikv.STATUS_BLOCK
    # writes through a bad entry are dropped: block 0 (and every other pool
    # row) keeps its contents, the rows of good entries land
    status.zero_()
    before = kp.clone()
    rows = rand(g, (n_kv, 8, D))
    ikv.append_paged(kp, rows, table, bt, 0, status=status)
    torch.cuda.synchronize()
    assert int(status.cpu()[0]) == ikv.STATUS_BLOCK
    want = before.clone()
    for t in range(n_kv):
        blk = int(table[t // bt])
        if blk < 6:
            want[blk * bt + t % bt] = rows[t]
    assert torch.equal(kp, want)
    # the fused decode append through a bad entry is dropped too
    status.zero_()
    before_k, before_v = kp.clone(), vp.clone()
    kn, vn = rand(g, (8, D)), rand(g, (8, D))
    # token 2 * bt + 5 is in the table's third block, whose entry is bad
    ikv.attn_decode_paged(q, kp, vp, table, bt, 2 * bt + 6, k_new=kn, v_new=vn, status=status)
    torch.cuda.synchronize()
    assert int(status.cpu()[0]) == ikv.STATUS_BLOCK
    assert torch.equal(kp, before_k) and torch.equal(vp, before_v)
    # a good table raises nothing
    status.zero_()
    good = torch.tensor([0, 1, 2, 3, 4], dtype=torch.int32, device=dev)
    ikv.attn_decode_paged(q, kp, vp, good, bt, n_kv, status=status)
    torch.cuda.synchronize()
    assert int(status.cpu()[0]) == 0


# ---------------------------------------------------------------------------
# the whole model on a paged cache
# ---------------------------------------------------------------------------

def test_paged_engine_matches_contiguous_and_oracle(dev, oracle_pool):
    from ikv import qwen3
    cfg = qwen3.Qwen3Config(n_layer=3, n_vocab=8192, n_ctx_train=4096)
    w = qwen3.synthetic_weights(cfg, synth.config_seed(0, 20))
    p1 = synth.uniform_ints(synth.config_seed(0, 21), 100, cfg.n_vocab)  # prefill over two blocks
    p2 = synth.uniform_ints(synth.config_seed(0, 22), 7, cfg.n_vocab)
    flat = qwen3.Qwen3Engine(cfg, 256)
    flat.set_weights(w)
    paged = qwen3.Qwen3Engine(cfg, 256, block_tokens=64)
    paged.set_weights(w)
    a1 = flat.generate(p1, 60)[0]
    b1 = paged.generate(p1, 60)[0]          # 159 tokens: three blocks per layer
    st = paged.last_stats()
    assert b1 == a1
    assert st["fused_rope_decode"] == cfg.n_layer and st["fused_append_decode"] == cfg.n_layer
    # every decode step replayed from a captured graph, the steps that open
    # a block (128) writing their table entries before the launch
    assert st["step_replays"] == 59 and st["step_captures"] >= 1
    paged.set_step_replay(False)
    assert paged.generate(p1, 60)[0] == a1 and paged.last_stats()["step_replays"] == 0
    paged.set_step_replay(True)
    # the next sequence gets the returned blocks in reverse order: a
    # non-identity block table, same tokens
    a2 = flat.generate(p2, 150)[0]
    b2 = paged.generate(p2, 150)[0]
    assert b2 == a2
    assert a2 == oracle.Qwen3Oracle(cfg, w, 256).generate(p2, 150)
    # every node on its own (unfused paged append, paged decode, paged prefill)
    paged.set_fusion(False)
    assert paged.generate(p1, 60)[0] == a1
    flat.close()
    paged.close()


def test_paged_engine_pool_too_small_fails_cleanly(dev):
    from ikv import qwen3
    cfg = qwen3.Qwen3Config(n_layer=2, n_vocab=4096, n_ctx_train=4096)
    eng = qwen3.Qwen3Engine(cfg, 512, block_tokens=64, pool_blocks=2)  # 128 tokens per layer
    eng.init_synthetic(3)
    assert len(eng.generate(list(range(1, 60)), 40)[0]) == 40       # 98 tokens fit
    with pytest.raises(ikv.IkvError):
        eng.generate(list(range(1, 100)), 40)                        # 138 do not
    assert len(eng.generate(list(range(1, 60)), 40)[0]) == 40       # blocks came back
    eng.close()


# ---------------------------------------------------------------------------
# the whole model on the HBM <-> host offload tier
# ---------------------------------------------------------------------------

def test_offload_engine_matches_hbm_cache(dev, oracle_pool):
    """Every layer of a step is held while the step runs, so a single
    sequence needs all its layers resident, and a new sequence's host copies
    hold no rows: its layers become resident with no transfer; same tokens.
    (Eviction, write-back and upload of written rows between sequences are
    checked by tests/cpp/test_engine.cpp --gpu.)"""
    from ikv import qwen3
    cfg = qwen3.Qwen3Config(n_layer=3, n_vocab=8192, n_ctx_train=4096)
    w = qwen3.synthetic_weights(cfg, synth.config_seed(0, 30))
    prompt = synth.uniform_ints(synth.config_seed(0, 31), 40, cfg.n_vocab)
    flat = qwen3.Qwen3Engine(cfg, 256)
    flat.set_weights(w)
    layer_bytes = 256 * 8 * 128 * 4 * 2
    off = qwen3.Qwen3Engine(cfg, 256, offload_hbm_bytes=3 * layer_bytes)
    off.set_weights(w)
    want = flat.generate(prompt, 30)[0]
    assert off.generate(prompt, 30)[0] == want
    st = off.kv_stats()
    assert st["page_ins"] == 0 and st["evictions"] == 0 and st["bytes_in"] == 0 and st["bytes_out"] == 0
    assert want == oracle.Qwen3Oracle(cfg, w, 256).generate(prompt, 30)
    # two layers of budget cannot hold a step's three: a clean error, no fault
    small = qwen3.Qwen3Engine(cfg, 256, offload_hbm_bytes=2 * layer_bytes)
    small.set_weights(w)
    with pytest.raises(ikv.IkvError):
        small.generate(prompt, 5)
    for e in (flat, off, small):
        e.close()


@pytest.mark.parametrize("budget_layers", [3, 4])
def test_offload_interleaved_sequences_page_and_keep_tokens(dev, oracle_pool, budget_layers):
    """Two sequences decoded in turn on a cache whose HBM budget holds one
    sequence's 3 layers (or 4 of the 6): every turn evicts the other
    sequence's layers (writing back the rows it appended) and uploads this
    one's committed rows, and each sequence's tokens stay those it gets
    alone, which the oracle pins."""
    from ikv import qwen3
    cfg = qwen3.Qwen3Config(n_layer=3, n_vocab=8192, n_ctx_train=4096)
    w = qwen3.synthetic_weights(cfg, synth.config_seed(0, 32))
    prompts = [synth.uniform_ints(synth.config_seed(0, 33 + i), 40, cfg.n_vocab) for i in range(2)]
    P, N, cap = 40, 24, 64
    want = [oracle.Qwen3Oracle(cfg, w, cap).generate(p, N) for p in prompts]
    flat = qwen3.Qwen3Engine(cfg, cap)
    flat.set_weights(w)
    assert [flat.generate(p, N)[0] for p in prompts] == want
    assert flat.generate_interleaved(prompts, N)[0] == want
    layer_bytes = cap * 8 * 128 * 4 * 2
    off = qwen3.Qwen3Engine(cfg, cap, offload_hbm_bytes=budget_layers * layer_bytes)
    off.set_weights(w)
    toks, t = off.generate_interleaved(prompts, N)
    assert toks == want
    st = off.kv_stats()
    # every decode turn after the first round pages the sequence back in
    assert st["page_ins"] >= (N - 1) * (6 - budget_layers) and st["evictions"] > 0
    assert st["bytes_in"] > 0 and st["bytes_out"] > 0
    # the rows moved are the committed ones: at most the whole sequence per layer
    assert st["bytes_in"] <= st["page_ins"] * (P + N) * 8 * 128 * 4 * 2
    assert t.tpot_s > 0
    for e in (flat, off):
        e.close()

