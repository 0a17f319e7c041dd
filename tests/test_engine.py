"""The C++ engine layer (tests/cpp/test_engine.cpp): the KV-cache transaction
state machine on the host, and the Qwen3 attention slice scheduled on the
HIP backend, checked against the oracle."""
import pathlib
import subprocess

import pytest

BIN = pathlib.Path(__file__).resolve().parent / "cpp" / "test_engine"


def run(mode):
    assert BIN.exists(), f"{BIN} not built (python -c 'import __graft_entry__ as g; g.build()')"
    p = subprocess.run([str(BIN), mode], capture_output=True, text=True, timeout=300)
    failed = [line for line in p.stdout.splitlines() if line.startswith("FAIL")]
    assert p.returncode == 0 and not failed, p.stdout[-4000:] + p.stderr[-2000:]
    return p.stdout


def test_engine_host_state_machine():
    out = run("--cpu")
    assert "PASS rope angle table bit-exact with the oracle" in out


@pytest.mark.gpu
def test_engine_attention_slice_on_hip_backend(dev):
    out = run("--gpu")
    assert "PASS fusions decode step 5" in out
    assert "PASS cache bit-exact, layer 1, decode step 5" in out
    assert "PASS offload: two sequences in one sequence's HBM, attention and caches exact at every switch" in out
    assert ("PASS offload: every switch wrote back only the rows written since the upload and uploaded only "
            "committed rows") in out
