#!/usr/bin/env python3
"""bench.py — decode KV-attention + KV append on one MI355X.

Workload (BASELINE.json config 1 at ctx 4096): the Qwen3-0.6B layer shape
(16 query heads, 8 KV heads, head_dim 128, F32). One step is one decode token
through all 28 layers: per layer, one fused launch that appends the new K/V
row at position ctx and attends over ctx+1 cached keys. The 28 layer caches
(28 x 32 MiB = 897 MiB) are distinct, so the working set is more than twice
the 256 MB Infinity Cache and the figure is HBM bandwidth, not MALL bandwidth.
The 28 launches of a step are captured once in a HIP graph and replayed.

Algorithmic bytes per launch (Qwen3-0.6B):  8192*L + 32768
    K and V history 2*4096*L, new k,v read 8192, new rows written 8192,
    q read 8192, output written 8192.
value = total algorithmic bytes / timed wall time (GB/s); roofline.achieved =
the same bytes / mean launch duration; peak = 8 TB/s.

Model level (extra.model): the whole Qwen3 graph on the HIP backend with
random-init weights (N(0, 0.02^2), norms 1.0) and uniform synthetic prompt
ids, greedy, no EOS stop — BASELINE configs 0 (Qwen3-0.6B, P=32, 128 tokens),
3 (Qwen3-0.6B, P=2048, 512 tokens) and 4 (Qwen3-8B, P=4096, 256 tokens) —
reporting TTFT and TPOT as benchmarks/cpu/bench.cpp:239-281 defines them and
the token checksum of that harness (c = c*131 + token). The CPU leg runs the
oracle (restated reference CPU backend) on config 0's weights and prompt for a
few tokens: its TPOT, and whether its tokens equal the GPU's.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
Prints ONE JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT / "infer-llm_amd"), str(ROOT / "oracle")]

METRIC = "decode KV-attn GB/s (% HBM peak) @ctx 4096; TPOT ms Qwen3-0.6B F32"
HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
N_HEAD, N_HEAD_KV, D, N_LAYER = 16, 8, 128, 28
TRAFFIC_FILE = ROOT / "profiles" / "decode_append_ctx4096_traffic.json"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_bytes(ctx, n_head=N_HEAD, n_head_kv=N_HEAD_KV, d=D):
    row = n_head_kv * d * 4
    return 2 * row * ctx + 2 * row + 2 * row + 2 * n_head * d * 4


def prefill_flops(p, n_head=N_HEAD, d=D):
    # unmasked (query, key) pairs x (QK^T + PV) = n_head * P(P+1)/2 * 4d
    return n_head * (p * (p + 1) // 2) * 4 * d


def seeded(ikv, config, index, shape):
    """Host float32 N(0, 1) samples of stream config_seed(config, index): the
    portable splitmix64 / Box-Muller stream of ikv.synth (multithreaded C++
    form), the same numbers for the GPU and the CPU legs."""
    from ikv import synth
    return ikv.synth_normal(synth.config_seed(config, index), shape, threads=16)


class DecodeRig:
    """n_layer layers of KV cache at one context length, launched through the
    C-ABI. Config 1 inputs: layer i's K and V caches are streams
    config_seed(1, 100 + i) and (1, 200 + i); q, k_new, v_new (the same for
    every layer) are (1, 300), (1, 301), (1, 302)."""

    def __init__(self, torch, ikv, ctx, n_layer=N_LAYER, n_head=N_HEAD, block_tokens=0):
        self.torch, self.ikv, self.ctx, self.n_layer = torch, ikv, ctx, n_layer
        self.n_head = n_head
        self.block_tokens = block_tokens  # > 0: paged pools with a shuffled block table
        dev = torch.device("cuda:0")
        q = torch.from_numpy(seeded(ikv, 1, 300, (n_head, D))).to(dev)
        kn = torch.from_numpy(seeded(ikv, 1, 301, (N_HEAD_KV, D))).to(dev)
        vn = torch.from_numpy(seeded(ikv, 1, 302, (N_HEAD_KV, D))).to(dev)
        self.layers = []
        for i in range(n_layer):
            kc = torch.from_numpy(seeded(ikv, 1, 100 + i, (ctx + 1, N_HEAD_KV, D))).to(dev)
            vc = torch.from_numpy(seeded(ikv, 1, 200 + i, (ctx + 1, N_HEAD_KV, D))).to(dev)
            self.layers.append(dict(kc=kc, vc=vc, q=q, kn=kn, vn=vn,
                                    out=torch.empty((n_head, D), device=dev)))
        if block_tokens:
            import numpy as np
            n_blocks = (ctx + 1 + block_tokens - 1) // block_tokens
            rng = np.random.default_rng(0x1F0000 + 1000 + block_tokens)
            for L in self.layers:
                pool_blocks = n_blocks + 4
                table = rng.permutation(pool_blocks)[:n_blocks].astype(np.int32)
                L["table"] = torch.tensor(table, device=dev)
                for name in ("kc", "vc"):
                    pool = torch.empty((pool_blocks * block_tokens, N_HEAD_KV, D), device=dev)
                    for b, blk in enumerate(table):
                        n = min(block_tokens, ctx + 1 - b * block_tokens)
                        pool[blk * block_tokens:blk * block_tokens + n] = \
                            L[name][b * block_tokens:b * block_tokens + n]
                    L[name] = pool
                L["pages"] = ikv.kv_pages(L["table"], block_tokens, L["kc"])
        self.ws = ikv.decode_workspace(n_head, N_HEAD_KV, D, ctx + 1, device=dev)
        self.ws_bytes = self.ws.numel() * 4
        self.lib = ikv.load()
        self.graph = None

    def step(self):
        s = self.torch.cuda.current_stream().cuda_stream
        n_kv = self.ctx + 1
        for L in self.layers:
            if self.block_tokens:
                import ctypes
                rc = self.lib.ikv_attn_decode_paged_f32(
                    L["q"].data_ptr(), L["kc"].data_ptr(), L["vc"].data_ptr(),
                    ctypes.byref(L["pages"]), L["kn"].data_ptr(), L["vn"].data_ptr(),
                    L["out"].data_ptr(), self.n_head, N_HEAD_KV, D, n_kv, 0.0, self.ws.data_ptr(),
                    self.ws_bytes, s)
            else:
                rc = self.lib.ikv_attn_decode_f32(
                    L["q"].data_ptr(), L["kc"].data_ptr(), L["vc"].data_ptr(), L["kn"].data_ptr(),
                    L["vn"].data_ptr(), L["out"].data_ptr(), self.n_head, N_HEAD_KV, D, n_kv, 0.0,
                    self.ws.data_ptr(), self.ws_bytes, s)
            if rc != 0:
                raise RuntimeError(f"decode returned {rc}")

    def capture(self):
        torch = self.torch
        self.step()  # eager reference for the graph check
        torch.cuda.synchronize()
        ref = [L["out"].clone() for L in self.layers]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.step()  # warm the capture stream
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        self.graph = g
        for _ in range(3):  # every replay must match the eager step bit for bit
            for L in self.layers:
                L["out"].zero_()
            g.replay()
            torch.cuda.synchronize()
            for L, r in zip(self.layers, ref):
                if not torch.equal(L["out"], r):
                    raise RuntimeError("graph replay differs from the eager step")

    def run(self, n):
        for _ in range(n):
            if self.graph is not None:
                self.graph.replay()
            else:
                self.step()

    def time(self, steps, warmup):
        torch = self.torch
        self.run(warmup)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        self.run(steps)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3  # seconds


def prefill_inputs(torch, ikv, p):
    """BASELINE config 2 inputs at prompt length p: raw Q, K, V from streams
    config_seed(2, 10 + p), (2, 20 + p), (2, 30 + p); Q and K then go through
    the qk-RMSNorm (weight 1.0, eps 1e-6) and RoPE (theta 1e6, positions
    0..p-1) of a Qwen3 layer on the device, as the model feeds attention."""
    import numpy as np
    dev = torch.device("cuda:0")
    q = torch.from_numpy(seeded(ikv, 2, 10 + p, (p, N_HEAD, D))).to(dev)
    k = torch.from_numpy(seeded(ikv, 2, 20 + p, (p, N_HEAD_KV, D))).to(dev)
    v = torch.from_numpy(seeded(ikv, 2, 30 + p, (p, N_HEAD_KV, D))).to(dev)
    s, c = ikv.rope_sincos_table(ikv.rope_theta_table(1e6, D, p))
    s, c = torch.from_numpy(s).to(dev), torch.from_numpy(c).to(dev)
    pos = torch.from_numpy(np.arange(p, dtype=np.int32)).to(dev)
    ones = torch.ones(D, device=dev)
    q = ikv.qk_norm_rope(q, ones, pos, 1e-6, s, c)
    k = ikv.qk_norm_rope(k, ones, pos, 1e-6, s, c)
    torch.cuda.synchronize()
    return q, k, v


def time_prefill(torch, ikv, p, reps):
    """Seconds per prefill launch: `reps` launches captured in one HIP graph
    and replayed (a Python launch loop is host-bound below ~10 us a launch)."""
    q, k, v = prefill_inputs(torch, ikv, p)
    out = torch.empty_like(q)

    def launches():
        for _ in range(reps):
            ikv.attn_prefill(q, k, v, 0, out=out)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launches()  # warm (and load the kernels) outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launches()
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / (5 * reps)


def prefill_only(torch, ikv, p, reps):
    """BASELINE config 2 at one prompt length: the append of p K and V rows
    into a 28-layer contiguous cache and the causal GQA prefill of p tokens,
    each timed over `reps` launches per layer with HIP events."""
    dev = torch.device("cuda:0")
    warm_clocks(torch, 1.0)
    t_pre = time_prefill(torch, ikv, p, reps)
    rows = torch.from_numpy(seeded(ikv, 2, 20 + p, (p, N_HEAD_KV, D))).to(dev)
    caches = [torch.empty((p, N_HEAD_KV, D), device=dev) for _ in range(N_LAYER)]
    for c in caches:
        ikv.append(c, rows)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        for c in caches:
            ikv.append(c, rows)
    e1.record()
    torch.cuda.synchronize()
    t_app = e0.elapsed_time(e1) / 1e3 / reps / N_LAYER
    nbytes = 2 * p * N_HEAD_KV * D * 4  # read and written once
    tf = prefill_flops(p) / t_pre / 1e12
    return {"prefill": {"P": p, "us": round(t_pre * 1e6, 2), "tflops": round(tf, 2),
                        "mfma_frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)},
            "append": {"rows": p, "us": round(t_app * 1e6, 2), "bytes": nbytes,
                       "gbs": round(nbytes / t_app / 1e9, 1),
                       "frac": round(nbytes / t_app / 1e9 / HBM_PEAK_GBS, 4)}}


# The projections of one prefill layer at BASELINE configs 3 and 4 (n_out, k,
# tokens): q, k/v, o, gate/up, down of Qwen3-0.6B at 2048 prompt tokens and
# of Qwen3-8B at 4096.
GEMM_SHAPES = [
    ("0.6B q", 2048, 1024, 2048), ("0.6B k/v", 1024, 1024, 2048), ("0.6B o", 1024, 2048, 2048),
    ("0.6B gate/up", 3072, 1024, 2048), ("0.6B down", 1024, 3072, 2048),
    ("8B q/o", 4096, 4096, 4096), ("8B k/v", 1024, 4096, 4096), ("8B gate/up", 12288, 4096, 4096),
    ("8B down", 4096, 12288, 4096),
]


def graph_us(torch, fn, reps):
    """us per call of fn, captured `reps` times in a HIP graph, 3 replays."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    # captured on the stream of the warm-up call (a split-K product allocates
    # its stream's workspace on its first call, outside capture)
    with torch.cuda.graph(g, stream=side):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(3):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (3 * reps)


def warm_clocks(torch, seconds=2.0):
    """~2 s of large products to bring the clocks up (the first product timed
    cold ran ~10% slow)."""
    import time
    a = torch.randn(4096, 4096, device="cuda:0")
    t0 = time.time()
    while time.time() - t0 < seconds:
        for _ in range(20):
            torch.mm(a, a)
        torch.cuda.synchronize()
    del a


def gemm_table(torch, ikv):
    """ikv.mul_mat (the MFMA GEMM from 2048 tokens on) against torch.mm (the
    vendor BLAS) at GEMM_SHAPES: each timed as a HIP graph of several
    launches, best of three alternated rounds, after warming the clocks."""
    dev = torch.device("cuda:0")
    warm_clocks(torch)

    rows = {}
    for name, n, k, m in GEMM_SHAPES:
        w = torch.randn(n, k, device=dev) * 0.02
        x = torch.randn(m, k, device=dev)
        out = torch.empty(m, n, device=dev)
        ref = torch.empty(m, n, device=dev)
        reps = 10 if n * k * m < 1e10 else 3
        ours, blas = [], []
        for _ in range(3):
            ours.append(graph_us(torch, lambda: ikv.mul_mat(w, x, out=out), reps))
            blas.append(graph_us(torch, lambda: torch.mm(x, w.t(), out=ref), reps))
        o, b = min(ours), min(blas)
        tf = 2 * n * k * m / o / 1e6
        rows[name] = {"n_out": n, "k": k, "tokens": m, "us": round(o, 1), "tflops": round(tf, 1),
                      "mfma_frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
                      "blas_us": round(b, 1), "vs_blas": round(o / b, 3),
                      "bit_equal_blas": bool(torch.equal(out, ref))}
        log(f"[bench] gemm {name}: {o:.1f} us ({tf:.1f} TF/s), torch.mm {b:.1f} us, "
            f"ratio {o / b:.3f}")
        del w, x, out, ref
        torch.cuda.empty_cache()
    return rows


# (name, n_out, k) of the Qwen3 projections
PROJECTIONS = [("0.6B q", 2048, 1024), ("0.6B k/v", 1024, 1024), ("0.6B o", 1024, 2048),
               ("0.6B gate/up", 3072, 1024), ("0.6B down", 1024, 3072),
               ("8B q/o", 4096, 4096), ("8B k/v", 1024, 4096), ("8B gate/up", 12288, 4096),
               ("8B down", 4096, 12288)]
GEMM_TILES = ["128x128", "64x64", "64x32", "32x64", "32x32"]


def gemm_sweep(torch, ikv, tokens=(65, 128, 256, 512, 1024, 2047)):
    """Every tile shape of the prefill GEMM (libikv_bench.so), each with K
    split 1-8 ways (up to 2048 workgroups), against torch.mm
    and ikv.mul_mat's own plan, on the Qwen3 projections at prompt lengths
    below the headline's: us per product (HIP graph of several launches,
    best of three rounds)."""
    import ctypes
    blib = ikv.load_bench()
    dev = torch.device("cuda:0")
    warm_clocks(torch)
    ws = torch.zeros((16 << 10) + (8 << 20), dtype=torch.uint8, device=dev)
    rows = []
    for name, n, k in PROJECTIONS:
        w = torch.randn(n, k, device=dev) * 0.02
        for m in tokens:
            x = torch.randn(m, k, device=dev)
            out = torch.empty(m, n, device=dev)
            ref = torch.empty(m, n, device=dev)
            reps = 10 if n * k * m < 1e10 else 3

            def tile_fn(t, sk):
                def f():
                    rc = blib.ikv_bench_gemm_nt_tile_f32(w.data_ptr(), x.data_ptr(), out.data_ptr(),
                                                         n, k, m, None, t, sk, ws.data_ptr(),
                                                         ws.numel(),
                                                         torch.cuda.current_stream().cuda_stream)
                    if rc:
                        raise RuntimeError(f"tile {t} split {sk}: {rc}")
                return f
            tile, split = ctypes.c_int(), ctypes.c_int()
            if blib.ikv_bench_gemm_plan(n, k, m, ctypes.byref(tile), ctypes.byref(split)):
                raise RuntimeError("gemm plan")
            row = {"proj": name, "n_out": n, "k": k, "tokens": m,
                   "plan": f"{GEMM_TILES[tile.value]}/s{split.value}"}
            row["torch_mm_us"] = round(min(graph_us(torch, lambda: torch.mm(x, w.t(), out=ref), reps)
                                           for _ in range(3)), 2)
            row["mul_mat_us"] = round(min(graph_us(torch, lambda: ikv.mul_mat(w, x, out=out), reps)
                                          for _ in range(3)), 2)
            row["mul_mat_vs_torch"] = round(row["mul_mat_us"] / row["torch_mm_us"], 3)
            cands = []
            for t, tname in enumerate(GEMM_TILES):
                if t == 0 and n % 128:
                    continue
                bm, bn = (int(v) for v in tname.split("x"))
                n_tiles = -(-m // bm) * (n // bn)
                cands.append((t, 1, tname))
                cands += [(t, sk, f"{tname}/s{sk}") for sk in (2, 3, 4, 5, 6, 8)
                          if k // 64 >= 4 * sk and n_tiles * sk <= 2048
                          and n_tiles * sk * bm * bn * 4 <= (8 << 20)]
            for t, sk, key in cands:
                row[key] = round(min(graph_us(torch, tile_fn(t, sk), reps) for _ in range(3)), 2)
            # again after the candidates (the clocks drift over a row)
            row["mul_mat_us"] = min(row["mul_mat_us"], round(min(
                graph_us(torch, lambda: ikv.mul_mat(w, x, out=out), reps) for _ in range(3)), 2))
            row["mul_mat_vs_torch"] = round(row["mul_mat_us"] / row["torch_mm_us"], 3)
            best = min((key for _, _, key in cands), key=lambda c: row[c])
            row["best"] = best
            row["best_vs_torch"] = round(row[best] / row["torch_mm_us"], 3)
            rows.append(row)
            log(f"[bench] sweep {name} m={m}: torch {row['torch_mm_us']} mul_mat {row['mul_mat_us']} "
                f"({row['plan']}) best {best} {row[best]}")
            del x, out, ref
        del w
        torch.cuda.empty_cache()
    return rows


def hbm_probes(torch, ikv):
    """What this box sustains, measured in the same run: a long streaming read
    (897 MiB per kernel), a streaming read of one decode layer's size (33.6 MB
    per kernel, 28 rotating buffers, HIP graph), and an empty kernel."""
    import ctypes

    lib = ikv.load_bench()
    dev = torch.device("cuda:0")
    sink = torch.empty(16384, device=dev)
    res = {}

    def timed_graph(fn, reps):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        g.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3 / reps

    def read(buf, grid, u):
        rc = lib.ikv_probe_read(buf.data_ptr(), buf.numel() * 4, sink.data_ptr(), grid, u,
                                torch.cuda.current_stream().cuda_stream)
        if rc:
            raise RuntimeError(f"ikv_probe_read {rc}")

    big = torch.ones(N_LAYER * decode_bytes(4096) // 4 // 16 * 16, device=dev)
    t = timed_graph(lambda: read(big, 2048, 8), 5)
    res["read_long_gbs"] = round(big.numel() * 4 / t / 1e9, 1)
    del big
    # one decode layer's bytes per launch, 28 distinct buffers (> 2x the MALL), in
    # grids shaped like decode's (208 workgroups of 512 threads at ctx 4096: 26 splits
    # x 8 KV heads; 256 = one per CU) and wider, with 1 to 16 loads in flight per lane;
    # the fastest is the floor one launch of this size reaches on this box
    bufs = [torch.ones(decode_bytes(4096) // 4 // 16 * 16, device=dev) for _ in range(N_LAYER)]
    shapes = {}
    for grid, u in ((208, 16), (256, 16), (256, 8), (528, 8), (1056, 4), (2048, 1)):
        t = timed_graph(lambda: [read(b, grid, u) for b in bufs], 10) / N_LAYER
        shapes[f"{grid}x512_u{u}"] = round(t * 1e6, 2)
    best = min(shapes, key=shapes.get)
    res["read_33MB_us"] = shapes
    res["read_33MB_floor_us"] = shapes[best]
    res["read_33MB_floor_shape"] = best
    res["read_33MB_floor_gbs"] = round(bufs[0].numel() * 4 / (shapes[best] * 1e-6) / 1e9, 1)
    del bufs

    def empties():
        for _ in range(200):
            lib.ikv_probe_empty(1024, torch.cuda.current_stream().cuda_stream)

    res["empty_kernel_us"] = round(timed_graph(empties, 5) / 200 * 1e6, 2)
    torch.cuda.empty_cache()
    return res


def paged_vs_contiguous(torch, ikv, ctx, steps, rounds=5):
    """Decode + append at ctx over 28 layers, contiguous and paged (64- and
    256-token blocks, shuffled tables), graph-replayed, the three rigs timed
    in alternation: GB/s of each round, and medians."""
    rigs = {"contiguous": DecodeRig(torch, ikv, ctx)}
    for bt in (64, 256):
        rigs[f"paged{bt}"] = DecodeRig(torch, ikv, ctx, block_tokens=bt)
    for r in rigs.values():
        r.capture()
        r.time(steps, 3)
    b = decode_bytes(ctx) * steps * N_LAYER
    res = {k: [] for k in rigs}
    for _ in range(rounds):
        for k, r in rigs.items():
            res[k].append(round(b / r.time(steps, 0) / 1e9, 1))
    out = {k: {"median_gbs": sorted(v)[len(v) // 2], "rounds_gbs": v} for k, v in res.items()}
    for k in ("paged64", "paged256"):
        out[k]["vs_contiguous"] = round(out[k]["median_gbs"] / out["contiguous"]["median_gbs"], 3)
    log(f"[bench] paged vs contiguous at ctx {ctx}: " +
        ", ".join(f"{k} {v['median_gbs']}" for k, v in out.items()))
    return out


def decode_timeline(torch, ikv, ctx=4096, n_head=N_HEAD, n_layer=N_LAYER, reps=30):
    """Phase timeline of one decode launch: the same workload as the headline
    (n_layer rotating caches at ctx, HIP graph), run through the stamped build
    of the decode kernels in libikv_bench.so. Each workgroup records the
    100 MHz s_memrealtime count at its entry, first tile scored, last tile
    scored (every wave), waves merged, partial published, arrival counted and
    (the merging workgroup) merge done; the records of the step's last launch
    are read after each of `reps` steps. Times are us from the launch's first
    workgroup entry, medians over the steps; the stamps add a little work, so
    the stamped launch runs slightly longer than the product one."""
    import ctypes
    import numpy as np
    blib = ikv.load_bench()
    rig = DecodeRig(torch, ikv, ctx, n_layer=n_layer, n_head=n_head)
    rig.lib = blib
    rig.capture()
    stamped_us = rig.time(20, 5) / 20 / n_layer * 1e6
    words = 1024 * 16
    recs = []
    for _ in range(reps):
        if blib.ikv_bench_timeline_clear() != 0:
            raise RuntimeError("ikv_bench_timeline_clear")
        rig.run(1)
        torch.cuda.synchronize()
        h = (ctypes.c_ulonglong * words)()
        if blib.ikv_bench_timeline_read(h, words) != 0:
            raise RuntimeError("ikv_bench_timeline_read")
        a = np.array(h, dtype=np.int64).reshape(1024, 16)
        recs.append(a[a[:, 0] > 0])
    del rig
    torch.cuda.empty_cache()

    def us(x):
        return round(float(x) / 100.0, 2)  # 100 MHz ticks -> us

    keys = ("first_entry_max", "first_tile_min", "first_tile_med", "first_tile_max",
            "stream_end_min", "stream_end_med", "stream_end_max", "slowest_wave_max",
            "wave_spread_med", "waves_merged_after_slowest_wave_med", "publish_med",
            "arrival_atomic_med", "merge_med", "merge_max", "last_merge_end")
    per = {k: [] for k in keys}
    for a in recs:
        t0 = a[:, 0].min()
        t = a[:, :7] - t0
        role = (a[:, 7] >> 8) & 0xFF
        waves = a[:, 8:16]
        wv = np.where(waves > 0, waves - t0, 0)
        slowest = wv.max(axis=1)
        fastest = np.where(waves > 0, wv, np.iinfo(np.int64).max).min(axis=1)
        split = role != 2
        m = role == 1
        per["first_entry_max"].append(t[:, 0].max())
        per["first_tile_min"].append(t[:, 1].min())
        per["first_tile_med"].append(np.median(t[:, 1]))
        per["first_tile_max"].append(t[:, 1].max())
        per["stream_end_min"].append(t[:, 2].min())
        per["stream_end_med"].append(np.median(t[:, 2]))
        per["stream_end_max"].append(t[:, 2].max())
        per["slowest_wave_max"].append(slowest.max())
        per["wave_spread_med"].append(np.median(slowest - fastest))
        per["waves_merged_after_slowest_wave_med"].append(np.median(t[:, 3] - slowest))
        if split.any():
            per["publish_med"].append(np.median(t[split, 4] - t[split, 3]))
            per["arrival_atomic_med"].append(np.median(t[split, 5] - t[split, 4]))
        if m.any():
            per["merge_med"].append(np.median(t[m, 6] - t[m, 5]))
            per["merge_max"].append((t[m, 6] - t[m, 5]).max())
            per["last_merge_end"].append(t[m, 6].max())
    out = {"ctx": ctx, "n_head": n_head, "workgroups": int(len(recs[-1])),
           "stamped_launch_us": round(stamped_us, 2)}
    for k, v in per.items():
        out[k + "_us"] = us(np.median(v)) if v else None
    # workgroup w = split * n_head_kv + kv head: do a KV head's splits share one XCD?
    xcc = (recs[-1][:, 7] & 15)
    n_kv_heads = N_HEAD_KV
    same = all(len(set(xcc[g::n_kv_heads].tolist())) == 1 for g in range(n_kv_heads))
    out["kv_head_splits_share_one_xcc"] = bool(same)
    return out


def pmc_per_dispatch(csv_path, kernel_substr):
    """Mean over dispatches of one counter (summed over its instances) for
    the kernels whose name contains kernel_substr, from a rocprofv3
    run_counter_collection.csv."""
    import collections
    import csv

    per = collections.defaultdict(float)
    with open(csv_path) as f:
        for r in csv.DictReader(f):
            if kernel_substr in r["Kernel_Name"]:
                per[r["Dispatch_Id"]] += float(r["Counter_Value"])
    if not per:
        raise SystemExit(f"no dispatch of *{kernel_substr}* in {csv_path}")
    return len(per), sum(per.values()) / len(per)


def traffic_summary(fetch_dir, write_dir, cal_fetch_dir, cal_write_dir, ctx):
    """HBM bytes per decode launch from two rocprofv3 --pmc runs (FETCH_SIZE,
    WRITE_SIZE, KiB per dispatch), each scaled by what the same counter reads
    for the --pmc-calibrate copy of known size (256 MiB read and written)."""
    csv_name = "run_counter_collection.csv"
    cal_bytes = 256 * 2**20
    n_f, fetch = pmc_per_dispatch(f"{fetch_dir}/{csv_name}", "decode_kernel")
    n_w, write = pmc_per_dispatch(f"{write_dir}/{csv_name}", "decode_kernel")
    _, cal_f = pmc_per_dispatch(f"{cal_fetch_dir}/{csv_name}", "copy")
    _, cal_w = pmc_per_dispatch(f"{cal_write_dir}/{csv_name}", "copy")
    f_factor = cal_bytes / (cal_f * 1024)
    w_factor = cal_bytes / (cal_w * 1024)
    fetch_b = fetch * 1024 * f_factor
    write_b = write * 1024 * w_factor
    return {
        "ctx": ctx,
        "workload": "ikv_attn_decode_f32 with fused append, Qwen3-0.6B layer shape (16 q heads, "
                    f"8 KV heads, head_dim 128), n_kv {ctx + 1}",
        "kernel": "decode_kernel<2>",
        "dispatches": {"fetch": n_f, "write": n_w},
        "fetch_kib_raw": round(fetch, 2),
        "write_kib_raw": round(write, 2),
        "fetch_bytes": round(fetch_b),
        "write_bytes": round(write_b),
        "hbm_bytes_per_launch": round(fetch_b + write_b),
        "algorithmic_bytes_per_launch": decode_bytes(ctx),
        "calibration": {"kernel": "ikv_append_f32 copy of 256 MiB (bench.py --pmc-calibrate)",
                        "fetch_kib_raw": round(cal_f, 2), "write_kib_raw": round(cal_w, 2),
                        "fetch_factor": round(f_factor, 5), "write_factor": round(w_factor, 5)},
    }


MODEL_CONFIGS = {  # (architecture, prompt, generated tokens)
    0: ("QWEN3_0_6B", 32, 128),
    3: ("QWEN3_0_6B", 2048, 512),
    4: ("QWEN3_8B", 4096, 256),
}


def token_checksum(tokens):
    c = 0
    for t in tokens:
        c = (c * 131 + (t & 0xFFFFFFFF)) & 0xFFFFFFFFFFFFFFFF
    return c


def model_bench(configs, cpu_tokens):
    """TTFT / TPOT of the whole model on the GPU per config, and the oracle's
    TPOT on config 0 (cpu_tokens greedy tokens) with a token-equality check."""
    from ikv import qwen3, synth

    res = {}
    gpu_tokens0 = None
    runs = []
    for c in configs:
        runs.append((c, 0))
        if c == 3:
            # config 3 again on a paged cache of 256-token blocks, right after
            # the contiguous run so that both see the same clocks
            runs.append((3, 256))
    for c, bt in runs:
        arch, P, N = MODEL_CONFIGS[c]
        cfg = getattr(qwen3, arch)
        t0 = time.perf_counter()
        eng = qwen3.Qwen3Engine(cfg, P + N, block_tokens=bt)
        eng.init_synthetic(synth.config_seed(c, 1), threads=16)
        init_s = time.perf_counter() - t0
        prompt = synth.uniform_ints(synth.config_seed(c, 0), P, cfg.n_vocab)
        # warm-up on the timed prompt (benchmarks/cpu/bench.cpp:414-431 warms up with
        # a whole run): arena, sin/cos tables, and every GEMM shape the prefill uses
        # (the library loads its kernels on first use)
        eng.generate(prompt, 4)
        # 3 timed runs, medians reported (benchmarks/cpu/bench.cpp:421-431)
        runs3 = [eng.generate(prompt, N) for _ in range(3)]
        toks = runs3[0][0]
        if any(r[0] != toks for r in runs3[1:]):
            raise RuntimeError(f"config {c}: repeated runs gave different tokens")
        t = sorted((r[1] for r in runs3), key=lambda x: x.tpot_s)[1]
        ttft_med = sorted(r[1].ttft_s for r in runs3)[1]
        st = eng.last_stats()
        eng.close()
        if c == 0:
            gpu_tokens0 = toks
        key = f"config{c}" + (f"_paged{bt}" if bt else "")
        res[key] = {
            "model": arch.lower().replace("_", "-").replace("-0-6b", "-0.6b"),
            "prompt": P, "generated": N, "ttft_ms": round(ttft_med * 1e3, 3),
            "tpot_ms": round(t.tpot_s * 1e3, 4), "decode_tok_s": round(1 / t.tpot_s, 1),
            "host_build_ms_per_step": round(t.build_s / N * 1e3, 4),
            "host_enqueue_ms_per_step": round(t.execute_s / N * 1e3, 4),
            "launches_per_decode_step": st["launches"], "token_checksum": str(token_checksum(toks)),
            "weights_gib": round(sum(int(__import__("numpy").prod(sh))
                                     for _, sh in qwen3.tensor_layout(cfg)) * 4 / 2**30, 2),
            "init_s": round(init_s, 1),
        }
        log(f"[bench] model config {c}{f' paged {bt}' if bt else ''} "
            f"({arch}, P={P}, N={N}): TTFT {ttft_med * 1e3:.2f} ms, TPOT {t.tpot_s * 1e3:.3f} ms "
            f"(medians of 3)")
    if cpu_tokens and 0 in configs:
        import oracle

        arch, P, _ = MODEL_CONFIGS[0]
        cfg = getattr(qwen3, arch)
        workers = min(oracle.default_workers(), 15)
        threads = oracle.set_workers(workers)
        w = qwen3.synthetic_weights(cfg, synth.config_seed(0, 1), threads=16)
        orc = oracle.Qwen3Oracle(cfg, w, P + cpu_tokens)
        prompt = synth.uniform_ints(synth.config_seed(0, 0), P, cfg.n_vocab)
        ids, n_past, times, toks = list(prompt), 0, [], []
        start = time.perf_counter()
        for _ in range(cpu_tokens):
            logits = orc.step(ids, n_past)
            tok = oracle.sample_greedy(logits[-1])
            times.append(time.perf_counter())
            toks.append(tok)
            n_past += len(ids)
            ids = [tok]
        res["cpu_config0"] = {
            "kind": "port", "threads": threads, "tokens": cpu_tokens,
            "ttft_ms": round((times[0] - start) * 1e3, 1),
            "tpot_ms": round((times[-1] - times[0]) / (cpu_tokens - 1) * 1e3, 2),
            "tokens_equal_gpu_prefix": gpu_tokens0 is not None and toks == gpu_tokens0[:cpu_tokens],
        }
        log(f"[bench] cpu config 0: TPOT {res['cpu_config0']['tpot_ms']} ms on {threads} threads, "
            f"tokens equal GPU: {res['cpu_config0']['tokens_equal_gpu_prefix']}")
        del w, orc
    if 0 in configs:
        res["published_profile"] = published_bench()
    if 3 in configs:
        res["config3_offload_2seq"] = offload_bench()
    return res


# The reference's published CUDA table (RTX 4060 Laptop, real Qwen3-0.6B
# weights): docs/performance/cuda-contiguous-kv-20261107/README.md:34-37.
PUBLISHED_REF = {32: (220.50, 17.94), 64: (423.20, 17.88), 128: (837.00, 24.68),
                 256: (1737.24, 28.12)}  # prompt -> (TTFT ms, TPOT ms)


def published_bench(prompts=(32, 64, 128, 256), n_gen=128):
    """The reference's published benchmark profile on this engine: Qwen3-0.6B
    F32 (config 0's synthetic weights), prompt ids (100 + i) % n_vocab
    (benchmarks/cpu/bench.cpp:393), 128 greedy tokens with no EOS stop, one
    warm-up and three timed runs per prompt length, mean and sample standard
    deviation of TTFT and TPOT as the reference's table reports them."""
    from ikv import qwen3, synth

    cfg = qwen3.QWEN3_0_6B
    res = {}
    for P in prompts:
        eng = qwen3.Qwen3Engine(cfg, P + n_gen)
        eng.init_synthetic(synth.config_seed(0, 1), threads=16)
        prompt = [(100 + i) % cfg.n_vocab for i in range(P)]
        eng.generate(prompt, n_gen)  # warm-up, a whole run
        runs = [eng.generate(prompt, n_gen) for _ in range(3)]
        eng.close()
        toks = runs[0][0]
        if any(r[0] != toks for r in runs[1:]):
            raise RuntimeError(f"published P={P}: repeated runs gave different tokens")
        ttft = [r[1].ttft_s * 1e3 for r in runs]
        tpot = [r[1].tpot_s * 1e3 for r in runs]
        ref_ttft, ref_tpot = PUBLISHED_REF.get(P, (None, None))
        res[f"P{P}"] = {
            "ttft_ms": round(statistics.mean(ttft), 3), "ttft_std_ms": round(statistics.stdev(ttft), 3),
            "tpot_ms": round(statistics.mean(tpot), 4), "tpot_std_ms": round(statistics.stdev(tpot), 4),
            "decode_tok_s": round(1e3 / statistics.mean(tpot), 1),
            "token_checksum": str(token_checksum(toks)),
            "reference_rtx4060_ttft_ms": ref_ttft, "reference_rtx4060_tpot_ms": ref_tpot,
        }
        log(f"[bench] published profile P={P}, N={n_gen}: TTFT {res[f'P{P}']['ttft_ms']} ms, "
            f"TPOT {res[f'P{P}']['tpot_ms']} ms (means of 3)")
    res["note"] = ("synthetic weights, so the tokens and checksums differ from the reference's "
                   "(real weights); its times are an RTX 4060 Laptop's")
    return res


HOST_LINK_GBS = 64.0  # PCIe 5.0 x16, one direction (the MI355X host link)


def offload_bench(n_gen=48):
    """Two config-3 sequences (Qwen3-0.6B, 2048-token prompts) decoded in
    turn, on the HBM <-> host offload tier with an HBM budget of ONE
    sequence's 28 layers, and on the all-HBM cache: every turn of the
    offloaded run writes back the other sequence's appended rows and uploads
    this one's committed rows (the reference's OffloadKVStorage under two
    sequences, include/kvcache/KVStorages/offloadKVStorage.hpp:57-179).
    Reports the bytes per run and the paging rate implied by the extra time
    per round over the all-HBM run, against the host link."""
    from ikv import qwen3, synth

    cfg = qwen3.QWEN3_0_6B
    P = MODEL_CONFIGS[3][1]
    cap = P + n_gen
    prompts = [synth.uniform_ints(synth.config_seed(3, 0), P, cfg.n_vocab),
               synth.uniform_ints(synth.config_seed(3, 2), P, cfg.n_vocab)]
    layer_bytes = cap * cfg.n_head_kv * cfg.head_dim * 4 * 2
    out = {"model": "qwen3-0.6b", "sequences": 2, "prompt": P, "generated": n_gen,
           "hbm_budget_bytes": cfg.n_layer * layer_bytes,
           "combined_layer_bytes": 2 * cfg.n_layer * layer_bytes}
    toks = {}
    for name, budget in (("hbm", 0), ("offload", cfg.n_layer * layer_bytes)):
        eng = qwen3.Qwen3Engine(cfg, cap, offload_hbm_bytes=budget)
        eng.init_synthetic(synth.config_seed(3, 1), threads=16)
        eng.generate_interleaved(prompts, 4)  # warm-up
        kv0 = eng.kv_stats()
        runs = [eng.generate_interleaved(prompts, n_gen) for _ in range(3)]
        kv1 = eng.kv_stats()
        eng.close()
        toks[name] = runs[0][0]
        if any(r[0] != toks[name] for r in runs[1:]):
            raise RuntimeError(f"offload bench ({name}): repeated runs gave different tokens")
        t = sorted((r[1] for r in runs), key=lambda x: x.tpot_s)[1]
        out[f"{name}_round_ms"] = round(t.tpot_s * 1e3, 3)
        out[f"{name}_ttft_ms"] = round(sorted(r[1].ttft_s for r in runs)[1] * 1e3, 2)
        if budget:
            out["kv_per_run"] = {k: (kv1[k] - kv0[k]) // 3 for k in kv1}
    if toks["hbm"] != toks["offload"]:
        raise RuntimeError("offload bench: the offloaded run's tokens differ from the all-HBM run's")
    kv = out["kv_per_run"]
    rounds = n_gen - 1
    extra_s = (out["offload_round_ms"] - out["hbm_round_ms"]) * 1e-3
    moved = (kv["bytes_in"] + kv["bytes_out"]) / max(rounds, 1)  # per round, both turns
    out["bytes_per_round"] = int(moved)
    out["tokens_equal_hbm"] = True
    if extra_s > 0:
        out["paging_gbs"] = round(moved / extra_s / 1e9, 1)
        out["paging_frac_host_link"] = round(moved / extra_s / 1e9 / HOST_LINK_GBS, 3)
    log(f"[bench] offload, 2 config-3 sequences in one sequence's HBM: round "
        f"{out['offload_round_ms']} ms vs {out['hbm_round_ms']} ms all-HBM, per run {kv}, "
        f"{out.get('paging_gbs')} GB/s paging")
    return out


def cpu_baseline(ctx, seconds):
    """The oracle (restated reference CPU backend) on this host: the same
    decode step (append + attention) of one layer, rotated over 8 layers."""
    import ikv
    import oracle

    workers = min(oracle.default_workers(), 15)
    threads = oracle.set_workers(workers)
    layers = []
    for i in range(8):  # the GPU rig's first 8 layer caches
        kc = seeded(ikv, 1, 100 + i, ((ctx + 1), N_HEAD_KV, D))
        vc = seeded(ikv, 1, 200 + i, ((ctx + 1), N_HEAD_KV, D))
        layers.append((kc, vc))
    q = seeded(ikv, 1, 300, (N_HEAD, D))
    kn = seeded(ikv, 1, 301, (N_HEAD_KV, D))
    vn = seeded(ikv, 1, 302, (N_HEAD_KV, D))
    oracle.decode_append_attn(q, kn, vn, *layers[0], ctx)  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        kc, vc = layers[n % len(layers)]
        oracle.decode_append_attn(q, kn, vn, kc, vc, ctx)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {
        "value": round(decode_bytes(ctx) * n / el / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{n} decode steps (append + GQA attention, 1 layer, ctx {ctx}) rotated over "
                  f"8 layer caches, {el:.1f} s; {workers} pool workers + calling thread "
                  f"(reference ThreadPool convention), host nproc {os.cpu_count()}",
        "ms_per_layer": round(el / n * 1e3, 3),
    }


def cpu_sweep():
    """The oracle on this host at every ctx of config 1 (decode step: append +
    attention, GB/s) and every prompt length of config 2 (prefill attention +
    append, ms), 1 warm-up and the median of 3 runs (benchmarks/cpu/bench.cpp
    :414-431)."""
    import numpy as np

    import ikv
    import oracle

    workers = min(oracle.default_workers(), 15)
    threads = oracle.set_workers(workers)

    def median3(fn):
        # a warm-up run, then 3 timed runs; a run longer than 0.5 s is warm
        # enough by itself, so its warm-up counts as the first timed run
        t0 = time.perf_counter()
        fn()
        first = time.perf_counter() - t0
        ts = [first] if first > 0.5 else []
        while len(ts) < 3:
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[1]

    res = {"threads": threads, "decode_gbs": {}, "prefill_ms": {}, "prefill_gflops": {}}
    q = seeded(ikv, 1, 300, (N_HEAD, D))
    kn = seeded(ikv, 1, 301, (N_HEAD_KV, D))
    vn = seeded(ikv, 1, 302, (N_HEAD_KV, D))
    for ctx in (256, 1024, 4096, 16384, 32768):
        kc = seeded(ikv, 1, 100, ((ctx + 1), N_HEAD_KV, D))
        vc = seeded(ikv, 1, 200, ((ctx + 1), N_HEAD_KV, D))
        t = median3(lambda: oracle.decode_append_attn(q, kn, vn, kc, vc, ctx))
        res["decode_gbs"][str(ctx)] = round(decode_bytes(ctx) / t / 1e9, 2)
        del kc, vc
    for P in (32, 64, 128, 256, 2048):
        # the GPU leg's inputs: the same streams, Q and K through the oracle's
        # qk-RMSNorm and RoPE (bit-identical to the device ops)
        th = oracle.rope_theta_table(1e6, D, P)
        pos = np.arange(P, dtype=np.int32)
        ones = np.ones(D, np.float32)

        def norm_rope(x):
            n = oracle.rms_norm(x.reshape(-1, D), ones, 1e-6).reshape(x.shape)
            return oracle.rope_neox(n, pos, th)
        qp = norm_rope(seeded(ikv, 2, 10 + P, (P, N_HEAD, D)))
        kp = norm_rope(seeded(ikv, 2, 20 + P, (P, N_HEAD_KV, D)))
        vp = seeded(ikv, 2, 30 + P, (P, N_HEAD_KV, D))
        kcache = np.empty_like(kp)
        vcache = np.empty_like(vp)

        def run():
            oracle.cpy(kcache, kp)
            oracle.cpy(vcache, vp)
            oracle.flash_attn(qp, kcache, vcache, 0)
        t = median3(run)
        res["prefill_ms"][str(P)] = round(t * 1e3, 3)
        res["prefill_gflops"][str(P)] = round(prefill_flops(P) / t / 1e9, 2)
    log(f"[bench] cpu sweep ({threads} threads): decode GB/s {res['decode_gbs']}, "
        f"prefill ms {res['prefill_ms']}")
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the ctx sweep and prefill")
    ap.add_argument("--eager", action="store_true", help="launch without HIP-graph capture")
    ap.add_argument("--model-configs", default="0,3,4",
                    help="BASELINE configs run at model level ('' for none)")
    ap.add_argument("--cpu-model-tokens", type=int, default=6,
                    help="greedy tokens the oracle generates on config 0 (0: skip)")
    ap.add_argument("--model-only", action="store_true",
                    help="only the model-level runs (--model-configs); prints their JSON")
    ap.add_argument("--traffic-from", nargs=4, metavar=("FETCH", "WRITE", "CAL_FETCH", "CAL_WRITE"),
                    help="summarise four rocprofv3 --pmc output folders into the traffic file "
                         "(no GPU needed)")
    ap.add_argument("--prefill-only", type=int, default=0, metavar="P",
                    help="only the prefill attention and the KV append of P prompt tokens "
                         "(BASELINE config 2 shape); prints their JSON (for counter runs)")
    ap.add_argument("--gemm-only", action="store_true",
                    help="only the prefill projection GEMMs of configs 3 and 4 against the "
                         "vendor BLAS; prints their JSON")
    ap.add_argument("--timeline-only", action="store_true",
                    help="only the decode phase timeline (stamped build, libikv_bench.so); "
                         "prints its JSON")
    ap.add_argument("--gemm-sweep", action="store_true",
                    help="only the prefill GEMM's tile shapes against torch.mm on the Qwen3 "
                         "projections below 2048 tokens; prints their JSON")
    ap.add_argument("--paged-only", action="store_true",
                    help="only decode at --ctx on contiguous and paged caches (5 alternated "
                         "rounds each); prints their JSON")
    ap.add_argument("--probes-only", action="store_true",
                    help="only the HBM / launch probes; prints their JSON")
    ap.add_argument("--pmc-calibrate", action="store_true",
                    help="only run 3 copies of 256 MiB through ikv_append_f32 (counter calibration)")
    args = ap.parse_args()
    if args.traffic_from:
        t = traffic_summary(*args.traffic_from, ctx=args.ctx)
        TRAFFIC_FILE.write_text(json.dumps(t, indent=1) + "\n")
        print(json.dumps(t))
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the hot path has no "
              "multi-GPU leg in this build", file=sys.stderr)
        sys.exit(2)

    import torch

    import ikv

    torch.cuda.set_device(0)
    ikv.load()
    if args.pmc_calibrate:
        n = 256 * 2**20
        a = torch.ones(n // 4, device="cuda:0")
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        for _ in range(3):
            ikv.append(b, a)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_calibration": "ikv_append_f32 copy", "bytes_read": n,
                          "bytes_written": n, "dispatches": 3}), flush=True)
        return
    log(f"[bench] {ikv.version()} on {torch.cuda.get_device_name(0)}")
    if args.probes_only:
        print(json.dumps(hbm_probes(torch, ikv)), flush=True)
        return
    if args.paged_only:
        print(json.dumps({"paged_vs_contiguous": paged_vs_contiguous(torch, ikv, args.ctx,
                                                                      args.steps)}), flush=True)
        return
    if args.timeline_only:
        print(json.dumps({"decode_timeline": [decode_timeline(torch, ikv, args.ctx),
                                              decode_timeline(torch, ikv, args.ctx, n_head=32,
                                                              n_layer=36)]}), flush=True)
        return
    if args.gemm_sweep:
        print(json.dumps({"gemm_sweep": gemm_sweep(torch, ikv)}), flush=True)
        return
    if args.gemm_only:
        print(json.dumps({"prefill_gemm": gemm_table(torch, ikv)}), flush=True)
        return
    if args.prefill_only:
        print(json.dumps(prefill_only(torch, ikv, args.prefill_only, args.steps)), flush=True)
        return
    if args.model_only:
        configs = [int(c) for c in args.model_configs.split(",") if c.strip()]
        print(json.dumps({"model": model_bench(configs, 0 if args.no_cpu else args.cpu_model_tokens)}),
              flush=True)
        return

    rig = DecodeRig(torch, ikv, args.ctx)
    if not args.eager:
        rig.capture()
        log(f"[bench] graph captured ({N_LAYER} launches per step), replays match eager")
    secs = rig.time(args.steps, args.warmup)
    launches = args.steps * N_LAYER
    per_launch = secs / launches
    bpl = decode_bytes(args.ctx)
    value = bpl * launches / secs / 1e9
    achieved = bpl / per_launch / 1e9
    log(f"[bench] ctx {args.ctx}: {secs / args.steps * 1e3:.3f} ms/step, "
        f"{per_launch * 1e6:.2f} us/launch, {value:.1f} GB/s")

    traffic = None
    if TRAFFIC_FILE.exists():
        t = json.loads(TRAFFIC_FILE.read_text())
        if t.get("ctx") == args.ctx:
            traffic = t.get("hbm_bytes_per_launch")

    extra = {"repeats": None, "eager_gbs": None, "ctx_sweep_gbs": {}, "short_ctx_us": {},
             "g4_ctx4096": None, "paged_ctx4096_gbs": {},
             "mall_hot_gbs": None, "prefill": {}, "prefill_gemm": None, "hbm_probes": None,
             "decode_timeline": None,
             "model": None,
             "cpu_sweep": None}
    if not args.no_extra:
        # Five more timed regions of the same K steps (no warmup between them):
        # their spread and median, beside the single region `value` reports.
        reps = sorted(bpl * launches / rig.time(args.steps, 0) / 1e9 for _ in range(5))
        extra["repeats"] = {"n": 5, "steps_each": args.steps, "median_gbs": round(reps[2], 1),
                            "min_gbs": round(reps[0], 1), "max_gbs": round(reps[-1], 1)}
        log(f"[bench] 5 repeats of {args.steps} steps: median {reps[2]:.1f} GB/s "
            f"(min {reps[0]:.1f}, max {reps[-1]:.1f})")
        rig.graph = None
        es = rig.time(max(args.steps // 2, 5), 2)
        extra["eager_gbs"] = round(bpl * max(args.steps // 2, 5) * N_LAYER / es / 1e9, 1)
        del rig
        torch.cuda.empty_cache()
        for ctx in (256, 1024, 4096, 16384, 32768):
            r = DecodeRig(torch, ikv, ctx)
            r.capture()
            n = max(5, min(50, int(2e4 // max(ctx // 64, 1))))
            s = r.time(n, 3)
            extra["ctx_sweep_gbs"][str(ctx)] = round(decode_bytes(ctx) * n * N_LAYER / s / 1e9, 1)
            log(f"[bench] sweep ctx {ctx}: {extra['ctx_sweep_gbs'][str(ctx)]} GB/s")
            del r
            torch.cuda.empty_cache()
        for ctx in (32, 96, 160, 512):  # the contexts of model config 0's decode steps
            r = DecodeRig(torch, ikv, ctx)
            r.capture()
            s = r.time(50, 3)
            extra["short_ctx_us"][str(ctx)] = round(s / 50 / N_LAYER * 1e6, 2)
            del r
        log(f"[bench] short contexts, us per layer: {extra['short_ctx_us']}")
        # the same workload on a paged cache (shuffled block tables)
        for bt in (64, 256):
            r = DecodeRig(torch, ikv, args.ctx, block_tokens=bt)
            r.capture()
            s = r.time(args.steps, 3)
            extra["paged_ctx4096_gbs"][str(bt)] = round(bpl * args.steps * N_LAYER / s / 1e9, 1)
            del r
        log(f"[bench] paged ctx {args.ctx}, GB/s by block size: {extra['paged_ctx4096_gbs']}")
        # Qwen3-8B layer shape (32 query heads over 8 KV heads, G = 4), 36 layers.
        r = DecodeRig(torch, ikv, 4096, n_layer=36, n_head=32)
        r.capture()
        s = r.time(20, 3)
        b = decode_bytes(4096, n_head=32)
        extra["g4_ctx4096"] = {"us": round(s / 20 / 36 * 1e6, 2),
                               "gbs": round(b * 20 * 36 / s / 1e9, 1)}
        log(f"[bench] G=4 ctx 4096: {extra['g4_ctx4096']}")
        del r
        torch.cuda.empty_cache()
        hot = DecodeRig(torch, ikv, args.ctx, n_layer=1)
        hot.layers = hot.layers * N_LAYER  # the same cache 28 times: MALL-resident
        hot.capture()
        s = hot.time(20, 3)
        extra["mall_hot_gbs"] = round(bpl * 20 * N_LAYER / s / 1e9, 1)
        del hot
        extra["hbm_probes"] = hbm_probes(torch, ikv)
        log(f"[bench] hbm probes: {extra['hbm_probes']}")
        extra["decode_timeline"] = decode_timeline(torch, ikv, args.ctx)
        log(f"[bench] decode timeline: {extra['decode_timeline']}")
        warm_clocks(torch, 1.0)
        for p in (32, 64, 128, 256, 2048):
            t = time_prefill(torch, ikv, p, 20 if p < 2048 else 10)
            tf = prefill_flops(p) / t / 1e12
            extra["prefill"][str(p)] = {"us": round(t * 1e6, 2), "tflops": round(tf, 2),
                                        "mfma_frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)}
            log(f"[bench] prefill P={p}: {t * 1e6:.1f} us, {tf:.2f} TFLOP/s")
        extra["prefill_gemm"] = gemm_table(torch, ikv)

    configs = [int(c) for c in args.model_configs.split(",") if c.strip()]
    if configs and not args.no_extra:
        torch.cuda.empty_cache()
        extra["model"] = model_bench(configs, 0 if args.no_cpu else args.cpu_model_tokens)

    cpu = None
    if not args.no_cpu:
        log(f"[bench] cpu baseline ({args.cpu_seconds:.0f} s)...")
        cpu = cpu_baseline(args.ctx, args.cpu_seconds)
        log(f"[bench] cpu baseline {cpu['value']} GB/s on {cpu['cores']} threads")
        if not args.no_extra:
            extra["cpu_sweep"] = cpu_sweep()

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(secs / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: K,V,q,k_new,v_new ~ N(0,1) F32 from the portable splitmix64 "
                "streams config_seed(1, 100+layer / 200+layer / 300..302), the CPU leg's data",
        "config": {
            "workload": "decode attention + fused KV append, Qwen3-0.6B layer shape "
                        f"(16 q heads, 8 KV heads, head_dim 128), n_past {args.ctx}, one step = "
                        f"{N_LAYER} layers with distinct caches ({N_LAYER} x "
                        f"{2 * (args.ctx + 1) * 4096 / 2**20:.0f} MiB), HIP-graph replay",
            "ctx": args.ctx, "layers": N_LAYER, "n_head": N_HEAD, "n_head_kv": N_HEAD_KV,
            "head_dim": D, "bytes_per_launch": bpl,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "launch_us": round(per_launch * 1e6, 3),
            # the fastest streaming read of one launch's bytes measured in this run
            # (extra.hbm_probes): the floor a kernel of this size reaches on this box
            "read_floor_us": (extra["hbm_probes"] or {}).get("read_33MB_floor_us")
            if args.ctx == 4096 else None,
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
