"""Greedy-token identity of the long model configurations on the HIP backend:
the engine's tokens at the full workloads of BASELINE configs 3 and 4 against
the fixtures the CPU oracle (the restated reference CPU backend) wrote in the
build container (tests/golden/make_model_tokens.py).

  config 3: Qwen3-0.6B architecture F32, 2048-token prompt, 512 greedy tokens
            (contiguous cache, paged cache of 256-token blocks, and the
            HBM <-> host offload tier)
  config 4: Qwen3-8B architecture F32, 4096-token prompt, 256 greedy tokens
  the reference's published profile: Qwen3-0.6B architecture F32 (config
            0's weights), prompts of 32 / 64 / 128 / 256 ids (100 + i) %
            n_vocab (benchmarks/cpu/bench.cpp:393), 128 greedy tokens

The reference treats one greedy stream as the correctness invariant of a KV
path: the same token checksum c = c*131 + token (benchmarks/cpu/bench.cpp:268)
for its CPU-no-KV, CPU-KV and CUDA-KV runs. A divergence is reported with its
first step and the oracle's top-1 / top-2 logit gap there, so that a near-tie
(a gap within float rounding of the logits) is told apart from a bug.

A greedy stream pins little once it settles on one token (config 3's repeats
one id from step 33 on), so the engine's logits are also checked at the
fixture's probe steps (0, 32, 128, 256, last): the oracle's eight largest
logits, ids and values, within |engine - oracle| <= 1e-3 + 1e-3 |oracle|.
"""
import json
import pathlib

import numpy as np
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


PUBLISHED = (32, 64, 128, 256)


def published_fixture(prompt_len):
    return json.loads((GOLDEN / f"qwen3_published_P{prompt_len}_tokens.json").read_text())


def fixture_prompt(fx, n_vocab):
    if fx.get("profile") == "published":
        return [(100 + i) % n_vocab for i in range(fx["prompt_len"])]
    return synth.uniform_ints(fx["prompt_seed"], fx["prompt_len"], n_vocab)


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


LOGIT_ATOL, LOGIT_RTOL = 1e-3, 1e-3


def probe_steps(fx):
    return sorted(int(s) for s in fx.get("logit_probes", {}))


def check_logits(logits, fx, what):
    """The engine's logits at the probe steps against the oracle's top 8."""
    for k, st in enumerate(probe_steps(fx)):
        p = fx["logit_probes"][str(st)]
        want = np.asarray(p["values"], np.float64)
        got = logits[k][p["ids"]].astype(np.float64)
        err = np.abs(got - want)
        print(f"{what} step {st}: top-8 max |diff| {err.max():.3e}", flush=True)
        assert np.all(err <= LOGIT_ATOL + LOGIT_RTOL * np.abs(want)), \
            f"{what} step {st}: logits {got} against the oracle's {want}"
        # and the engine's own largest logit is the oracle's top id
        assert int(np.argmax(logits[k])) == p["ids"][0], f"{what} step {st}: argmax"


def run_engine(fx, **kw):
    cfg = getattr(qwen3, fx["model"])
    P, N = fx["prompt_len"], fx["n_gen"]
    eng = qwen3.Qwen3Engine(cfg, P + N, **kw)
    try:
        eng.init_synthetic(fx["weight_seed"], std=fx["std"], threads=16)
        prompt = fixture_prompt(fx, cfg.n_vocab)
        steps = probe_steps(fx)
        if steps:
            eng.capture_logits(steps)
        toks, _ = eng.generate(prompt, N)
        logits = eng.captured_logits() if steps else None
        stats = eng.kv_stats() if kw.get("offload_hbm_bytes") else None
    finally:
        eng.close()
    return toks, stats, logits


def test_fixtures_follow_the_benchmark_seeds():
    for c, (arch, P, N) in {3: ("QWEN3_0_6B", 2048, 512), 4: ("QWEN3_8B", 4096, 256)}.items():
        fx = fixture(c)
        assert (fx["model"], fx["prompt_len"], fx["n_gen"]) == (arch, P, N)
        assert fx["weight_seed"] == synth.config_seed(c, 1)
        assert fx["prompt_seed"] == synth.config_seed(c, 0)
        assert len(fx["tokens"]) == len(fx["top2_gap"]) == N
        assert str(checksum(fx["tokens"])) == fx["token_checksum"]
        steps = probe_steps(fx)
        assert steps == sorted({s for s in (0, 32, 128, 256, N - 1) if s < N})
        for s in steps:  # the probe's top id is the step's greedy token
            assert fx["logit_probes"][str(s)]["ids"][0] == fx["tokens"][s]


def test_published_fixtures_follow_the_reference_profile():
    for P in PUBLISHED:
        fx = published_fixture(P)
        assert (fx["model"], fx["prompt_len"], fx["n_gen"]) == ("QWEN3_0_6B", P, 128)
        assert fx["weight_seed"] == synth.config_seed(0, 1) and fx["std"] == 0.02
        assert fx["prompt"] == "(100+i) % n_vocab"
        assert len(fx["tokens"]) == len(fx["top2_gap"]) == 128
        assert str(checksum(fx["tokens"])) == fx["token_checksum"]
        assert probe_steps(fx) == [0, 32, 127]
        for s in probe_steps(fx):
            assert fx["logit_probes"][str(s)]["ids"][0] == fx["tokens"][s]


@pytest.mark.gpu
@pytest.mark.parametrize("prompt_len", PUBLISHED)
def test_published_profile_greedy_tokens_match_oracle(dev, prompt_len):
    # prefills of 32 and 64 tokens run the few-token MFMA kernel, 128 and 256
    # the tiled GEMM (K split for the narrow projections at 128)
    fx = published_fixture(prompt_len)
    toks, _, logits = run_engine(fx)
    check_stream(toks, fx, f"published profile P={prompt_len}")
    check_logits(logits, fx, f"published profile P={prompt_len}")


@pytest.mark.gpu
def test_config3_greedy_tokens_match_oracle(dev):
    fx = fixture(3)
    toks, _, logits = run_engine(fx)
    check_stream(toks, fx, "config 3, contiguous cache")
    check_logits(logits, fx, "config 3, contiguous cache")


@pytest.mark.gpu
def test_config3_paged_greedy_tokens_match_oracle(dev):
    fx = fixture(3)
    toks, _, logits = run_engine(fx, block_tokens=256)
    check_stream(toks, fx, "config 3, paged cache (256-token blocks)")
    check_logits(logits, fx, "config 3, paged cache")


@pytest.mark.gpu
def test_config3_offload_greedy_tokens_match_oracle(dev):
    # the offload tier with an HBM budget of exactly the sequence's layers
    # (a step holds all its layers): the caches live in pinned host memory
    # copies managed by the tier, and the tokens must not change
    fx = fixture(3)
    cfg = qwen3.QWEN3_0_6B
    layer_bytes = (fx["prompt_len"] + fx["n_gen"]) * cfg.n_head_kv * cfg.head_dim * 4 * 2
    toks, _, logits = run_engine(fx, offload_hbm_bytes=cfg.n_layer * layer_bytes)
    check_stream(toks, fx, "config 3, offload tier")
    check_logits(logits, fx, "config 3, offload tier")


@pytest.mark.gpu
def test_config4_greedy_tokens_match_oracle(dev):
    fx = fixture(4)
    toks, _, logits = run_engine(fx)
    check_stream(toks, fx, "config 4 (Qwen3-8B), contiguous cache")
    check_logits(logits, fx, "config 4 (Qwen3-8B), contiguous cache")
