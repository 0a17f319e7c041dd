"""The committed fixtures (tests/golden/hotpath_small.npz) against the oracle
and their float64 references, on the CPU."""
import pathlib

import numpy as np
import pytest

import oracle

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "hotpath_small.npz"


@pytest.fixture(scope="module")
def g():
    oracle.set_workers(1)
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_oracle_reproduces_fixtures_bitwise(g):
    assert np.array_equal(bits(oracle.rms_norm(g["rms_x"], g["rms_w"], 1e-6)), bits(g["rms_out"]))
    th = oracle.rope_theta_table(1e6, 128, 4096)
    assert np.array_equal(bits(oracle.rope_neox(g["rms_out"], g["rope_pos"], th)), bits(g["rope_out"]))
    assert np.array_equal(bits(oracle.flash_attn(g["dec_q"], g["dec_k"], g["dec_v"], 16)), bits(g["dec_out"]))
    assert np.array_equal(bits(oracle.flash_attn(g["pre_q"], g["pre_k"], g["pre_v"], 0)), bits(g["pre_out"]))


def test_fixture_outputs_agree_with_float64(g):
    for a, b in (("rms_out", "rms_out_f64"), ("dec_out", "dec_out_f64"), ("pre_out", "pre_out_f64")):
        err = np.abs(g[a].astype(np.float64) - g[b])
        assert np.all(err <= 1e-6 + 1e-5 * np.abs(g[b])), a
