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
c = c*131 + token (benchmarks/cpu/bench.cpp:268).

Usage (tens of minutes for config 4; its weights take 28.2 GiB of RAM):
  python tests/golden/make_model_tokens.py --config 3 4 [--workers 7]
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
HERE = pathlib.Path(__file__).resolve().parent


def fixture_path(config: int) -> pathlib.Path:
    return HERE / f"qwen3_config{config}_tokens.json"


def checksum(tokens) -> int:
    c = 0
    for t in tokens:
        c = (c * 131 + (t & 0xFFFFFFFF)) & 0xFFFFFFFFFFFFFFFF
    return c


def run(config: int, n_gen: int | None = None, log=print) -> dict:
    arch, P, N = CONFIGS[config]
    N = N if n_gen is None else n_gen
    cfg = getattr(qwen3, arch)
    t0 = time.time()
    w = qwen3.synthetic_weights(cfg, synth.config_seed(config, 1), threads=8)
    prompt = synth.uniform_ints(synth.config_seed(config, 0), P, cfg.n_vocab)
    orc = oracle.Qwen3Oracle(cfg, w, P + N)
    log(f"config {config}: weights ready in {time.time() - t0:.0f} s")
    ids, n_past = list(prompt), 0
    tokens, runner_up, gaps = [], [], []
    for i in range(N):
        ts = time.time()
        row = orc.step(ids, n_past)[-1]
        tok = oracle.sample_greedy(row)
        if tok < 0:
            raise RuntimeError(f"config {config} step {i}: sampler rejected the logits")
        second = row.copy()
        second[tok] = -np.inf
        r = int(np.argmax(second))
        tokens.append(tok)
        runner_up.append(r)
        gaps.append(float(row[tok]) - float(row[r]))
        n_past += len(ids)
        ids = [tok]
        if i == 0 or (i + 1) % 32 == 0:
            log(f"config {config}: step {i + 1}/{N} token {tok} gap {gaps[-1]:.3g} "
                f"({time.time() - ts:.1f} s)")
    return {
        "config": config, "model": arch, "prompt_len": P, "n_gen": N,
        "weight_seed": synth.config_seed(config, 1), "prompt_seed": synth.config_seed(config, 0),
        "std": 0.02, "tokens": tokens, "runner_up": runner_up, "top2_gap": gaps,
        "token_checksum": str(checksum(tokens)),
        "oracle_threads": oracle_threads, "seconds": round(time.time() - t0, 1),
    }


oracle_threads = 1

if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", type=int, nargs="+", default=[3, 4])
    ap.add_argument("--workers", type=int, default=7)
    a = ap.parse_args()
    oracle_threads = oracle.set_workers(a.workers)
    for c in a.config:
        fx = run(c, log=lambda *m: print(*m, flush=True))
        fixture_path(c).write_text(json.dumps(fx) + "\n")
        print(f"wrote {fixture_path(c)} (checksum {fx['token_checksum']}, min gap "
              f"{min(fx['top2_gap']):.3g})", flush=True)
