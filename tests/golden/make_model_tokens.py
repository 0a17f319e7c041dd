"""Writes the greedy-token fixtures of the long model configurations from the
CPU oracle (the restated reference CPU backend), run in the build container:

  config 3: Qwen3-0.6B architecture F32, 2048-token prompt, 512 greedy tokens
  config 4: Qwen3-8B architecture F32, 4096-token prompt, 256 greedy tokens

Weights and prompt use the benchmark's seeds: matrices N(0, 0.02^2) from
synth.config_seed(c, 1) (norm weights 1.0), prompt ids uniform in
[0, n_vocab) from synth.config_seed(c, 0). The generation loop is the
reference benchmark's (benchmarks/cpu/bench.cpp:239-281: prefill, then one
token per step, no EOS stop, greedy with ties to the lower id,
src/sampler.cpp:42-65). For each step the fixture keeps the token, the
runner-up id and the top-1 minus top-2 logit gap, so that a GPU run that
diverges can tell a near-tie from a bug, and the reference's token checksum
c = c*131 + token (benchmarks/cpu/bench.cpp:268). At the steps of
probe_steps() it also keeps the eight largest logits (ids and values), which
pin the engine at logit level where a greedy stream alone pins little (a
stream that repeats one token shows only that a fixed point stays put).

It also writes the fixtures of the reference's published benchmark profile
(docs/performance/cuda-contiguous-kv-20261107/README.md: Qwen3-0.6B F32,
prompts of 32 / 64 / 128 / 256 tokens, 128 generated, prompt ids
(100 + i) % n_vocab as benchmarks/cpu/bench.cpp:393 builds them), on config
0's synthetic weights (synth.config_seed(0, 1)).

Usage (tens of minutes for config 4; its weights take 28.2 GiB of RAM):
  python tests/golden/make_model_tokens.py --config 3 4 [--workers 7]
  python tests/golden/make_model_tokens.py --config --published 32 64 128 256
"""
from __future__ import annotations

import argparse
import json
import pathlib
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "infer-llm_amd"))

import oracle  # noqa: E402
from ikv import qwen3, synth  # noqa: E402

CONFIGS = {3: ("QWEN3_0_6B", 2048, 512), 4: ("QWEN3_8B", 4096, 256)}
PUBLISHED_PROMPTS = (32, 64, 128, 256)
PUBLISHED_N = 128
HERE = pathlib.Path(__file__).resolve().parent


def fixture_path(config: int) -> pathlib.Path:
    return HERE / f"qwen3_config{config}_tokens.json"


def published_path(prompt_len: int) -> pathlib.Path:
    return HERE / f"qwen3_published_P{prompt_len}_tokens.json"


def published_prompt(prompt_len: int, n_vocab: int) -> list[int]:
    """benchmarks/cpu/bench.cpp:393: prompt[i] = (100 + i) % vocab."""
    return [(100 + i) % n_vocab for i in range(prompt_len)]


def probe_steps(n_gen: int) -> list[int]:
    """The steps whose logits the fixture keeps: 0, 32, 128, 256 and the last."""
    return sorted({s for s in (0, 32, 128, 256, n_gen - 1) if 0 <= s < n_gen})


TOP_K = 8


def checksum(tokens) -> int:
    c = 0
    for t in tokens:
        c = (c * 131 + (t & 0xFFFFFFFF)) & 0xFFFFFFFFFFFFFFFF
    return c


def run(config: int, n_gen: int | None = None, log=print) -> dict:
    arch, P, N = CONFIGS[config]
    N = N if n_gen is None else n_gen
    cfg = getattr(qwen3, arch)
    prompt = synth.uniform_ints(synth.config_seed(config, 0), P, cfg.n_vocab)
    fx = generate(arch, synth.config_seed(config, 1), prompt, N, f"config {config}", log)
    return {"config": config, "prompt_seed": synth.config_seed(config, 0), **fx}


def run_published(prompt_len: int, weights=None, log=print) -> dict:
    cfg = qwen3.QWEN3_0_6B
    fx = generate("QWEN3_0_6B", synth.config_seed(0, 1), published_prompt(prompt_len, cfg.n_vocab),
                  PUBLISHED_N, f"published P={prompt_len}", log, weights)
    return {"profile": "published", "prompt": "(100+i) % n_vocab", **fx}


def generate(arch, weight_seed, prompt, N, name, log, w=None) -> dict:
    cfg = getattr(qwen3, arch)
    P = len(prompt)
    t0 = time.time()
    if w is None:
        w = qwen3.synthetic_weights(cfg, weight_seed, threads=8)
    orc = oracle.Qwen3Oracle(cfg, w, P + N)
    log(f"{name}: weights ready in {time.time() - t0:.0f} s")
    ids, n_past = list(prompt), 0
    tokens, runner_up, gaps = [], [], []
    probes = {}
    keep = set(probe_steps(N))
    for i in range(N):
        ts = time.time()
        row = orc.step(ids, n_past)[-1]
        tok = oracle.sample_greedy(row)
        if tok < 0:
            raise RuntimeError(f"{name} step {i}: sampler rejected the logits")
        second = row.copy()
        second[tok] = -np.inf
        r = int(np.argmax(second))
        tokens.append(tok)
        runner_up.append(r)
        gaps.append(float(row[tok]) - float(row[r]))
        if i in keep:
            top = np.argsort(-row.astype(np.float64), kind="stable")[:TOP_K]
            probes[str(i)] = {"ids": [int(t) for t in top],
                              "values": [float(row[t]) for t in top]}
        n_past += len(ids)
        ids = [tok]
        if i == 0 or (i + 1) % 32 == 0:
            log(f"{name}: step {i + 1}/{N} token {tok} gap {gaps[-1]:.3g} "
                f"({time.time() - ts:.1f} s)")
    return {
        "model": arch, "prompt_len": P, "n_gen": N, "weight_seed": weight_seed,
        "std": 0.02, "tokens": tokens, "runner_up": runner_up, "top2_gap": gaps,
        "logit_probes": probes,
        "token_checksum": str(checksum(tokens)),
        "oracle_threads": oracle_threads, "seconds": round(time.time() - t0, 1),
    }


oracle_threads = 1

if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", type=int, nargs="*", default=[3, 4])
    ap.add_argument("--published", type=int, nargs="*", default=[])
    ap.add_argument("--workers", type=int, default=7)
    a = ap.parse_args()
    oracle_threads = oracle.set_workers(a.workers)
    if a.published:
        w0 = qwen3.synthetic_weights(qwen3.QWEN3_0_6B, synth.config_seed(0, 1), threads=8)
        for P in a.published:
            fx = run_published(P, w0, log=lambda *m: print(*m, flush=True))
            published_path(P).write_text(json.dumps(fx) + "\n")
            print(f"wrote {published_path(P)} (checksum {fx['token_checksum']}, min gap "
                  f"{min(fx['top2_gap']):.3g})", flush=True)
    for c in a.config:
        fx = run(c, log=lambda *m: print(*m, flush=True))
        fixture_path(c).write_text(json.dumps(fx) + "\n")
        print(f"wrote {fixture_path(c)} (checksum {fx['token_checksum']}, min gap "
              f"{min(fx['top2_gap']):.3g})", flush=True)
