"""The publish protocols of the in-kernel merges, checked in the gfx950 code
this build's compiler emits (CPU only: hipcc cross-compiles to assembly).

The split decode (attn_decode.hip: decode_kernel, qkv_attn_kernel), the
split-K GEMM (gemm.hip: gemm_nt_kernel) and the multi-workgroup sampler
(model_ops.hip: argmax_ws_kernel) publish partial
results with agent-coherent stores and then count their workgroup in an
arrival counter with a relaxed agent-scope atomic; the workgroup that counts
last reads every partial back. What makes that correct on gfx950 is the code
between the two: the stores carry the coherence bit (sc1), and a
`s_waitcnt vmcnt(0)` (CDNA counts stores in vmcnt) comes after the last of
them and before the atomic, and so does the workgroup barrier where several
wavefronts store and one counts (qkv_attn_kernel, gemm_nt_kernel; in decode_kernel one
wavefront stores every partial and counts). A release fence would express
the same order in the HIP memory model, but on this chip it writes back the
L2 (measured ~6 us per launch), so the kernels rely on the emitted order
instead, and this test pins it: a compiler that moved the atomic above the
wait, or dropped sc1 from the stores, fails here before it can corrupt a
merge on the GPU.
"""
import pathlib
import re
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
CSRC = ROOT / "infer-llm_amd" / "csrc"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
# the kernel flags of infer-llm_amd/Makefile (HIPFLAGS), device code only
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++20", "-DNDEBUG", "-Xclang", "-target-feature",
         "-Xclang", "-packed-fp32-ops", "-Wno-unused-command-line-argument", "--cuda-device-only",
         "-S"]

STORE_SC1 = re.compile(r"^\s*(global|buffer)_store\w*\b.*\bsc1\b")
WAIT_VM0 = re.compile(r"^\s*s_waitcnt\b.*\bvmcnt\(0\)")
BARRIER = re.compile(r"^\s*s_barrier\b")
ATOMIC_RET = re.compile(r"^\s*global_atomic_add\w*\b.*\bsc0\b")


def device_asm(src: pathlib.Path, tmp_path) -> str:
    if not pathlib.Path(HIPCC).exists():
        pytest.skip("hipcc not available")
    out = tmp_path / (src.stem + ".s")
    subprocess.run([HIPCC, *FLAGS, "-I", str(CSRC), "-I", str(ROOT / "include"), "-o", str(out),
                    str(src)], check=True, capture_output=True)
    return out.read_text()


def functions(asm: str):
    """(mangled name, body lines) of every kernel in the assembly."""
    name, body = None, []
    for line in asm.splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            name, body = m.group(1), []
            continue
        if name and line.startswith(".Lfunc_end"):
            yield name, body
            name = None
            continue
        if name:
            body.append(line)


def check_publish_order(name, body, many_writers=True):
    atomics = [i for i, l in enumerate(body) if ATOMIC_RET.match(l)]
    assert atomics, f"{name}: no arrival atomic found"
    for a in atomics:
        stores = [i for i in range(a) if STORE_SC1.match(body[i])]
        assert stores, f"{name}: no agent-coherent (sc1) partial store before the atomic"
        last = stores[-1]
        between = body[last + 1:a]
        assert any(WAIT_VM0.match(l) for l in between), \
            f"{name}: no s_waitcnt vmcnt(0) between the last sc1 store and the atomic"
        if many_writers:  # every thread's stores, then one thread counts
            assert any(BARRIER.match(l) for l in between), \
                f"{name}: no workgroup barrier between the last sc1 store and the atomic"


def test_split_decode_publishes_before_counting(tmp_path):
    asm = device_asm(CSRC / "attn_decode.hip", tmp_path)
    checked = 0
    for name, body in functions(asm):
        if "decode_kernel" in name:
            check_publish_order(name, body, many_writers=False)  # wave 0 stores and counts
            checked += 1
        elif "qkv_attn_kernel" in name:
            check_publish_order(name, body)
            checked += 1
    # decode_kernel<G, PRO, PAGED> for G in 1, 2, 4, 8 and qkv_attn_kernel<G>
    assert checked == 4 * 4 + 4


def test_split_k_gemm_publishes_before_counting(tmp_path):
    asm = device_asm(CSRC / "gemm.hip", tmp_path)
    found = [(n, b) for n, b in functions(asm) if "gemm_nt_kernel" in n]
    assert len(found) == 5  # the five tile shapes
    for name, body in found:
        check_publish_order(name, body)  # every thread stores its partial, one counts


def test_sampler_publishes_before_counting(tmp_path):
    asm = device_asm(CSRC / "model_ops.hip", tmp_path)
    found = [(n, b) for n, b in functions(asm) if "argmax_ws_kernel" in n]
    assert len(found) == 1
    check_publish_order(*found[0], many_writers=False)  # one thread stores and counts


def test_checker_catches_planted_mistakes():
    good = ["\tglobal_store_dword v[2:3], v1, off sc1", "\ts_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0)",
            "\ts_barrier", "\tglobal_atomic_add v3, v3, v4, s[4:5] sc0"]
    check_publish_order("good", good)
    moved = [good[0], good[3], good[1], good[2]]          # the atomic above the wait
    plain = ["\tglobal_store_dword v[2:3], v1, off"] + good[1:]  # no coherence bit
    no_barrier = [good[0], good[1], good[3]]
    for body in (moved, plain, no_barrier):
        with pytest.raises(AssertionError):
            check_publish_order("planted", body)
    check_publish_order("one writer", no_barrier, many_writers=False)
