"""Greedy-token identity of the long model configurations on the HIP backend:
the engine's tokens at the full workloads of BASELINE configs 3 and 4 against
the fixtures the CPU oracle (the restated reference CPU backend) wrote in the
build container (tests/golden/make_model_tokens.py).

  config 3: Qwen3-0.6B architecture F32, 2048-token prompt, 512 greedy tokens
            (contiguous cache, paged cache of 256-token blocks, and the
            HBM <-> host offload tier)
  config 4: Qwen3-8B architecture F32, 4096-token prompt, 256 greedy tokens

The reference treats one greedy stream as the correctness invariant of a KV
path: the same token checksum c = c*131 + token (benchmarks/cpu/bench.cpp:268)
for its CPU-no-KV, CPU-KV and CUDA-KV runs. A divergence is reported with its
first step and the oracle's top-1 / top-2 logit gap there, so that a near-tie
(a gap within float rounding of the logits) is told apart from a bug.
"""
import json
import pathlib

import pytest

from ikv import qwen3, synth

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def checksum(tokens):
    c = 0
    for t in tokens:
        c = (c * 131 + (t & 0xFFFFFFFF)) & 0xFFFFFFFFFFFFFFFF
    return c


def fixture(config):
    return json.loads((GOLDEN / f"qwen3_config{config}_tokens.json").read_text())


def check_stream(toks, fx, what):
    ref = fx["tokens"]
    if toks == ref:
        assert str(checksum(toks)) == fx["token_checksum"]
        return
    i = next(k for k, (a, b) in enumerate(zip(toks, ref)) if a != b) if len(toks) == len(ref) else -1
    gap = fx["top2_gap"][i] if i >= 0 else float("nan")
    runner = fx["runner_up"][i] if i >= 0 else None
    raise AssertionError(
        f"{what}: greedy stream diverges from the oracle at step {i} of {len(ref)}: "
        f"engine token {toks[i] if i >= 0 else None}, oracle token {ref[i] if i >= 0 else None} "
        f"(oracle runner-up {runner}, top-1 minus top-2 logit gap {gap:.3g})")


def run_engine(fx, **kw):
    cfg = getattr(qwen3, fx["model"])
    P, N = fx["prompt_len"], fx["n_gen"]
    eng = qwen3.Qwen3Engine(cfg, P + N, **kw)
    try:
        eng.init_synthetic(fx["weight_seed"], std=fx["std"], threads=16)
        prompt = synth.uniform_ints(fx["prompt_seed"], P, cfg.n_vocab)
        toks, _ = eng.generate(prompt, N)
        stats = eng.kv_stats() if kw.get("offload_hbm_bytes") else None
    finally:
        eng.close()
    return toks, stats


def test_fixtures_follow_the_benchmark_seeds():
    for c, (arch, P, N) in {3: ("QWEN3_0_6B", 2048, 512), 4: ("QWEN3_8B", 4096, 256)}.items():
        fx = fixture(c)
        assert (fx["model"], fx["prompt_len"], fx["n_gen"]) == (arch, P, N)
        assert fx["weight_seed"] == synth.config_seed(c, 1)
        assert fx["prompt_seed"] == synth.config_seed(c, 0)
        assert len(fx["tokens"]) == len(fx["top2_gap"]) == N
        assert str(checksum(fx["tokens"])) == fx["token_checksum"]


@pytest.mark.gpu
def test_config3_greedy_tokens_match_oracle(dev):
    fx = fixture(3)
    toks, _ = run_engine(fx)
    check_stream(toks, fx, "config 3, contiguous cache")


@pytest.mark.gpu
def test_config3_paged_greedy_tokens_match_oracle(dev):
    fx = fixture(3)
    toks, _ = run_engine(fx, block_tokens=256)
    check_stream(toks, fx, "config 3, paged cache (256-token blocks)")


@pytest.mark.gpu
def test_config3_offload_greedy_tokens_match_oracle(dev):
    # the offload tier with an HBM budget of exactly the sequence's layers
    # (a step holds all its layers): the caches live in pinned host memory
    # copies managed by the tier, and the tokens must not change
    fx = fixture(3)
    cfg = qwen3.QWEN3_0_6B
    layer_bytes = (fx["prompt_len"] + fx["n_gen"]) * cfg.n_head_kv * cfg.head_dim * 4 * 2
    toks, _ = run_engine(fx, offload_hbm_bytes=cfg.n_layer * layer_bytes)
    check_stream(toks, fx, "config 3, offload tier")


@pytest.mark.gpu
def test_config4_greedy_tokens_match_oracle(dev):
    fx = fixture(4)
    toks, _ = run_engine(fx)
    check_stream(toks, fx, "config 4 (Qwen3-8B), contiguous cache")
