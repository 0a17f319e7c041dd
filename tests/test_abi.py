"""The C-ABI library on the CPU: it loads, exports every entry point that
include/ikv.h declares, and rejects bad arguments before touching a device.
No kernel is launched here."""
import ctypes
import errno
import re
import subprocess

import numpy as np
import pytest

import ikv
import oracle


def test_library_loads_and_reports_version():
    assert ikv.version().startswith("ikv ")


def test_every_declared_entry_point_is_exported():
    declared = ikv.header_functions()
    assert declared, "no declarations parsed from include/ikv.h"
    lib = ikv.load()
    for name in declared:
        assert hasattr(lib, name), name
    exported = subprocess.run(["nm", "-D", "--defined-only", str(ikv.LIB_PATH)],
                              capture_output=True, text=True, check=True).stdout
    names = {line.split()[-1] for line in exported.splitlines() if line.strip()}
    assert set(declared) <= names
    from ikv import qwen3
    assert set(ikv.SIGNATURES) | set(qwen3.ENGINE_SIGNATURES) == set(declared)


def test_measurement_code_lives_in_the_bench_library():
    # libikv.so exports the path's ABI only; the probes and the stamped decode
    # build are in libikv_bench.so, which bench.py loads beside it
    def exported(path):
        out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True,
                             text=True, check=True).stdout
        return {line.split()[-1] for line in out.splitlines() if line.strip()}

    product = exported(ikv.LIB_PATH)
    assert not {n for n in product if n.startswith(("ikv_probe_", "ikv_bench_"))}
    text = re.sub(r"/\*.*?\*/", "", ikv.BENCH_HEADER.read_text(), flags=re.S)
    declared = set(re.findall(r"\b(ikv_[a-z0-9_]+)\s*\(", text))
    assert declared == set(ikv.BENCH_SIGNATURES)
    bench = exported(ikv.BENCH_LIB_PATH)
    assert declared <= bench
    assert "ikv_attn_decode_f32" in bench  # the stamped decode build
    ikv.load_bench()


def test_library_links_no_vendor_blas():
    # every product runs on this library's own kernels
    deps = subprocess.run(["ldd", str(ikv.LIB_PATH)], capture_output=True, text=True).stdout
    assert "rocblas" not in deps and "hipblas" not in deps


GEMM_TILE_NAMES = ["128x128", "64x64", "64x32", "32x64", "32x32"]


@pytest.mark.parametrize("n_out,k,m,plan", [
    # Qwen3-0.6B o_proj and Qwen3-8B k/v projections at 128 tokens: 128
    # tiles of 32 x 32, K split in two (256 workgroups, one per CU)
    (1024, 2048, 128, "32x32/2"), (1024, 4096, 128, "32x32/2"),
    (1024, 3072, 65, "32x32/5"),     # 96 tiles, 48 steps: 480 workgroups in 2 rounds
    (2048, 1024, 128, "32x32/1"),    # 256 tiles: one per CU
    (3072, 1024, 512, "64x32/1"),    # 768 tiles: whole rounds (64 x 64 would leave a half round)
    (4096, 4096, 512, "64x64/1"),
    (1024, 1024, 2048, "64x64/1"),   # 128 tiles of 128 x 128 would idle half the CUs
    (2048, 1024, 2048, "128x128/1"), (4096, 12288, 4096, "128x128/1"),
    (64, 4096, 300, "32x32/8"),      # 20 tiles: at most 8 splits
    (1024, 256, 65, "32x32/1"),      # 4 steps of 64 columns: too short to split
])
def test_gemm_plan(n_out, k, m, plan):
    import ctypes
    tile, split = ctypes.c_int(), ctypes.c_int()
    assert ikv.load_bench().ikv_bench_gemm_plan(n_out, k, m, ctypes.byref(tile),
                                                ctypes.byref(split)) == 0
    assert f"{GEMM_TILE_NAMES[tile.value]}/{split.value}" == plan


def test_library_does_not_link_the_oracle():
    deps = subprocess.run(["ldd", str(ikv.LIB_PATH)], capture_output=True, text=True).stdout
    assert "oracle" not in deps
    syms = subprocess.run(["nm", "-D", str(ikv.LIB_PATH)], capture_output=True, text=True).stdout
    assert "oracle_" not in syms


def _rc(name, *args):
    return getattr(ikv.load(), name)(*args)


def test_decode_rejects_bad_arguments_without_launching():
    P = 64  # fake 16-byte aligned non-null "device" address; never dereferenced
    ok = dict(n_head=16, n_head_kv=8, head_dim=128, n_kv=100)

    def call(q=P, k=P, v=P, kn=None, vn=None, out=P, n_head=16, n_head_kv=8, head_dim=128,
             n_kv=100, ws=None, wsb=0):
        return _rc("ikv_attn_decode_f32", q, k, v, kn, vn, out, n_head, n_head_kv, head_dim, n_kv,
                   0.0, ws, wsb, None)

    assert call(q=None) == -errno.EINVAL
    assert call(kn=P) == -errno.EINVAL                 # k_new without v_new
    assert call(n_head=12) == -errno.EINVAL            # not a multiple of n_head_kv
    assert call(n_kv=0) == -errno.EINVAL
    assert call(head_dim=1024) == -errno.ENOTSUP       # past the generic path's 512
    assert call(n_head=24, head_dim=640) == -errno.ENOTSUP
    # other head sizes and groups take the generic path: its workspace holds
    # the rotated q and k rows of the fused prologue (each 256-byte aligned),
    # then the split partials: (max, sum) records, 256-byte aligned, and
    # head_dim floats per query head and split. Splits: at least 64 keys
    # each, at most ceil(256 / n_head_kv).
    def a256(b):
        return (b + 255) // 256 * 256

    def generic(n_head, n_head_kv, d, n_splits):
        pro = a256(n_head * d * 4) + a256(n_head_kv * d * 4)
        return pro + a256(2 * n_head * n_splits * 4) + n_head * n_splits * d * 4

    assert ikv.decode_workspace_bytes(24, 8, 64, 100) == generic(24, 8, 64, 2)
    assert ikv.decode_workspace_bytes(12, 4, 96, 5000) == generic(12, 4, 96, 64)
    assert ikv.decode_workspace_bytes(12, 4, 96, 64) == generic(12, 4, 96, 1)
    # G * ceil(head_dim / 64) > 32 (dims per lane 1, 2, 4, 8): no split form
    assert ikv.decode_workspace_bytes(12, 2, 300, 5000) == a256(12 * 300 * 4) + a256(2 * 300 * 4)
    assert call(q=P + 4) == -errno.EINVAL              # misaligned
    assert call(n_kv=4097) == -errno.EINVAL            # split-K needs a workspace
    need = ikv.decode_workspace_bytes(ok["n_head"], ok["n_head_kv"], 128, 4097)
    assert call(n_kv=4097, ws=P, wsb=need - 4) == -errno.EINVAL


def test_noalloc_decode_rejects_shapes_before_touching_a_device():
    P = 64
    m = re.search(r"#define IKV_DECODE_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)",
                  (ikv.HEADER_DIR / "ikv.h").read_text())
    assert m and int(m[1]) << int(m[2]) == ikv.NOALLOC_SCRATCH_BYTES
    for name in ("POSITION", "BLOCK", "TOKEN"):
        m = re.search(rf"#define IKV_STATUS_{name} (\d+)", (ikv.HEADER_DIR / "ikv.h").read_text())
        assert m and int(m[1]) == getattr(ikv, f"STATUS_{name}")

    def call(n_head, n_head_kv, head_dim=128, n_kv=4097):
        return _rc("ikv_attn_decode_noalloc_f32", P, P, P, None, None, P, n_head, n_head_kv,
                   head_dim, n_kv, 0.0, None)

    # 4096 query heads over 512 KV heads: 2.26 MB of partials, more than the array
    assert ikv.decode_workspace_bytes(4096, 512, 128, 4097) > ikv.NOALLOC_SCRATCH_BYTES
    assert call(4096, 512) == -errno.ENOSPC
    assert call(12, 8) == -errno.EINVAL
    assert call(16, 8, n_kv=0) == -errno.EINVAL
    assert call(16, 8, head_dim=64) == -errno.ENOTSUP
    assert call(24, 8) == -errno.ENOTSUP              # group of 3
    assert call(16, 8, n_kv=2**31) == -errno.EOVERFLOW
    # every supported group size of up to 128 KV heads fits, at any context
    for hkv in (1, 8, 64, 128):
        for G in (1, 2, 4, 8):
            for n_kv in (129, 4097, 40960, 1 << 20):
                assert ikv.decode_workspace_bytes(hkv * G, hkv, 128, n_kv) <= ikv.NOALLOC_SCRATCH_BYTES


def test_qkv_attn_rejects_bad_arguments_without_launching():
    P = 64

    def call(n_head=16, n_head_kv=8, head_dim=128, n_kv=100, n_embd=1024, ptr=P, ws=P):
        return _rc("ikv_qkv_attn_decode_f32", ptr, P, P, P, None, 0.0, P, P, P, n_embd, P, P, P,
                   n_head, n_head_kv, head_dim, n_kv, 0.0, P, P, 1e-6, P, P, P, 10, None, ws,
                   1 << 20, None)

    assert call(n_kv=129) == -errno.ENOTSUP          # more than one decode split
    assert call(n_embd=1000) == -errno.ENOTSUP       # not a multiple of 1024
    assert call(ptr=None) == -errno.EINVAL
    assert call(ws=None) == -errno.EINVAL
    assert call(n_head=24) == -errno.ENOTSUP
    assert call(head_dim=64) == -errno.ENOTSUP
    assert call(n_kv=0) == -errno.EINVAL


def test_gemm_rejects_bad_arguments_without_launching():
    P, U = 64, 68  # 16-byte aligned, unaligned addresses

    def call(n_out=128, k=128, m=100, w=P, x=P, out=P):
        return _rc("ikv_gemm_nt_f32", w, x, out, n_out, k, m, None, None)

    assert call(n_out=100) == -errno.ENOTSUP      # n_out % 64
    assert call(k=96) == -errno.ENOTSUP           # k % 64
    assert call(k=0) == -errno.ENOTSUP
    assert call(w=U) == -errno.EINVAL             # unaligned weights
    assert call(x=U) == -errno.EINVAL
    assert call(out=None) == -errno.EINVAL
    assert call(m=-1) == -errno.EINVAL
    assert call(m=0) == 0 and call(n_out=0) == 0  # nothing to do
    assert call(m=2**40) == -errno.EOVERFLOW
    assert call(k=2**22) == -errno.ENOTSUP        # a 128-row panel past 32-bit offsets


def decode_ws_bytes(n_head, n_head_kv, n_splits):
    """The decode workspace of n_splits splits: one 256-byte counter slot per
    KV head, then one (max, sum) pair and one 128-float output per (query
    head, split), the regions 256-byte aligned."""
    a256 = lambda b: (b + 255) // 256 * 256  # noqa: E731
    return a256(256 * n_head_kv) + a256(8 * n_head * n_splits) + 4 * 128 * n_head * n_splits


def test_decode_plan_stays_within_one_workgroup_per_cu():
    # (host arithmetic) the workspace size tells the split count. The plan
    # never goes past 256 workgroups (32 splits x 8 KV heads): a 33rd split
    # per head put a second full split on some CUs, which then set the
    # kernel's end. ctx 4096 (4097 keys) takes 26 splits of 5 tiles.
    for n_head in (16, 32):
        ws = lambda n: ikv.decode_workspace_bytes(n_head, 8, 128, n)  # noqa: E731
        peak = ws(2048)  # 32 splits of 64 keys
        assert peak == decode_ws_bytes(n_head, 8, 32)
        assert all(ws(n) <= peak for n in range(129, 50001, 3))
        assert ws(20000) == peak and ws(40000) == peak
        assert ws(4097) == decode_ws_bytes(n_head, 8, 26)


def test_decode_replay_limit_tracks_the_split_plan():
    # (host arithmetic) Qwen3-0.6B shape: one split up to 128 keys, then
    # 64-key splits up to 32 per KV head (2048 keys), then 96-key splits
    lim = lambda n, w: ikv.decode_replay_limit(16, 8, 128, n, w)
    assert lim(1, 256) == 128 and lim(33, 256) == 128 and lim(128, 256) == 128
    assert lim(129, 256) == 384 and lim(129, 1) == 129
    assert lim(2000, 256) == 2048 and lim(2048, 256) == 2048
    assert lim(2049, 256) == 2304 and lim(2113, 256) == 2368
    # the plan the limit promises to keep: per-context workspace sizes grow
    # with the context and never pass the limit's
    for n in (129, 1000, 2113, 4000):
        m = lim(n, 256)
        need = ikv.decode_workspace_bytes(16, 8, 128, m)
        assert all(ikv.decode_workspace_bytes(16, 8, 128, x) <= need for x in range(n, m + 1, 37))
    assert lim(0, 256) == 0 and lim(100, 0) == 0
    assert ikv.decode_replay_limit(16, 8, 64, 100, 256) == 0  # head_dim the decode rejects


def test_replay_entries_reject_bad_arguments():
    P = 64
    assert _rc("ikv_attn_decode_rope_replay_f32", P, P, P, P, P, P, 16, 8, 128, 0, 0.0, P, P,
               1e-6, P, P, P, 10, None, P, 1 << 20, None) == -errno.EINVAL       # n_kv_max 0
    assert _rc("ikv_attn_decode_rope_replay_f32", P, P, P, P, P, P, 16, 8, 128, 100, 0.0, P, P,
               1e-6, None, P, P, 10, None, P, 1 << 20, None) == -errno.EINVAL    # no pos
    assert _rc("ikv_qkv_attn_decode_replay_f32", P, P, P, P, None, 0.0, P, P, P, 1024, P, P, P,
               16, 8, 128, 129, 0.0, P, P, 1e-6, P, P, P, 10, None, P, 1 << 20,
               None) == -errno.ENOTSUP                                         # two splits


def test_prefill_and_rows_reject_bad_arguments():
    P = 64
    assert _rc("ikv_attn_prefill_f32", P, P, P, P, 16, 8, 128, 0, 10, 0, 0.0, None) == 0  # n_q=0
    assert _rc("ikv_attn_prefill_f32", None, P, P, P, 16, 8, 128, 4, 10, 0, 0.0, None) == -errno.EINVAL
    assert _rc("ikv_attn_prefill_f32", P, P, P, P, 16, 8, 1024, 4, 10, 0, 0.0, None) == -errno.ENOTSUP
    # the MFMA kernel's tile rows (n_head_kv x 512 bytes) take 32-bit offsets
    assert _rc("ikv_attn_prefill_f32", P, P, P, P, 1 << 17, 1 << 17, 128, 4, 10, 0, 0.0,
               None) == -errno.EOVERFLOW
    assert _rc("ikv_rms_norm_f32", None, P, P, 4, 128, 1e-6, None) == -errno.EINVAL
    assert _rc("ikv_rms_norm_f32", P, P, P, 0, 128, 1e-6, None) == 0
    assert _rc("ikv_rope_neox_f32", P, P, P, 2, 8, 127, P, P, 10, None, None) == -errno.EINVAL
    assert _rc("ikv_qk_norm_rope_f32", P, None, P, P, 2, 8, 128, 1e-6, P, P, 10, None, None) == -errno.EINVAL
    assert _rc("ikv_append_f32", None, P, 1, 4096, None) == -errno.EINVAL
    assert _rc("ikv_append_f32", P, P, 0, 4096, None) == 0
    assert _rc("ikv_append_f32", P, P, 2**62, 2**8, None) == -errno.EOVERFLOW


def test_argmax_workspace_form_rejects_bad_arguments():
    P, W = 64, 256  # 16-byte aligned logits, 256-byte aligned workspace addresses
    need = ikv.load().ikv_argmax_workspace_bytes()
    assert 256 < need <= 4096
    assert _rc("ikv_argmax_ws_f32", P, 10, P, None, None, need, None) == -errno.EINVAL   # no workspace
    assert _rc("ikv_argmax_ws_f32", P, 10, P, None, W, need - 8, None) == -errno.EINVAL  # too small
    assert _rc("ikv_argmax_ws_f32", P, 10, P, None, W + 8, need, None) == -errno.EINVAL  # misaligned
    assert _rc("ikv_argmax_ws_f32", P, 0, P, None, W, need, None) == -errno.EINVAL       # n < 1
    assert _rc("ikv_argmax_ws_f32", None, 10, P, None, W, need, None) == -errno.EINVAL


def test_workspace_bytes_grow_with_context_and_are_bounded():
    sizes = [ikv.decode_workspace_bytes(16, 8, 128, n) for n in (1, 256, 4097, 32769, 10**6)]
    assert all(s > 0 for s in sizes)
    assert sizes == sorted(sizes)
    assert sizes[-1] <= 16 * 1024 * (128 + 2) * 4 + 4096  # at most 1024 splits per head
    # the generic path: prologue rows, then two splits' partials at 100 keys
    assert ikv.decode_workspace_bytes(16, 8, 64, 100) == (16 + 8) * 64 * 4 + 256 + 16 * 2 * 64 * 4
    # and its workspace too grows with the context and stops at 256 / n_head_kv splits
    gen = [ikv.decode_workspace_bytes(16, 8, 64, n) for n in (1, 100, 4097, 10**6)]
    assert gen == sorted(gen) and gen[-1] == gen[-2] == (16 + 8) * 64 * 4 + 2 * 16 * 32 * 4 + 16 * 32 * 64 * 4
    assert ikv.decode_workspace_bytes(16, 8, 1024, 100) == 0


def test_sincos_table_is_bitwise_glibc():
    """The host table must hold exactly the cosf/sinf values the reference CPU
    rope uses. The oracle's rope of unit vectors exposes them bitwise:
    e_j -> (cos, sin) at (j, j+64), since 1*c - 0*s == c exactly."""
    th = oracle.rope_theta_table(1e6, 128, 40960)
    pos = np.array([0, 1, 2, 1000, 4096, 32768, 40959], np.int32)
    s, c = ikv.rope_sincos_table(th[pos])
    x = np.zeros((len(pos), 64, 128), np.float32)
    x[:, np.arange(64), np.arange(64)] = 1.0
    r = oracle.rope_neox(x, pos, th)
    cos_ref = r[:, np.arange(64), np.arange(64)]
    sin_ref = r[:, np.arange(64), np.arange(64) + 64]
    assert np.array_equal(c.view(np.uint32), cos_ref.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), sin_ref.view(np.uint32))


@pytest.mark.parametrize("base,hd,n_ctx", [(1e6, 128, 40960), (1e4, 64, 300), (5e5, 2, 17)])
def test_theta_table_equals_the_oracle_bitwise(base, hd, n_ctx):
    # the product's angle table (the engine and the benchmark build theirs
    # with it) against the oracle's restatement of src/graph.cpp:92-135
    got = ikv.rope_theta_table(base, hd, n_ctx)
    want = oracle.rope_theta_table(base, hd, n_ctx)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert _rc("ikv_rope_theta_table_f32", 1e6, 127, 10, None) == -errno.EINVAL
    assert _rc("ikv_rope_theta_table_f32", 1e6, 128, 0, None) == 0


def test_paged_entry_points_reject_bad_descriptors():
    P = 64
    good = ikv.KvPages(P, 64, 10, None)
    bad_bt = ikv.KvPages(P, 48, 10, None)          # not a multiple of 64
    no_table = ikv.KvPages(None, 64, 10, None)
    huge = ikv.KvPages(P, 2**30, 2**20, None)     # pool rows beyond int
    ref = ctypes.byref

    def dec(pg):
        return _rc("ikv_attn_decode_paged_f32", P, P, P, pg, None, None, P, 16, 8, 128, 60, 0.0,
                   None, 0, None)

    assert dec(None) == -errno.EINVAL
    assert dec(ref(bad_bt)) == -errno.EINVAL
    assert dec(ref(no_table)) == -errno.EINVAL
    assert dec(ref(huge)) == -errno.EOVERFLOW
    assert _rc("ikv_attn_prefill_paged_f32", P, P, P, None, P, 16, 8, 128, 4, 10, 0, 0.0,
               None) == -errno.EINVAL
    assert _rc("ikv_attn_prefill_paged_f32", P, P, P, ref(bad_bt), P, 16, 8, 128, 4, 10, 0, 0.0,
               None) == -errno.EINVAL
    assert _rc("ikv_append_paged_f32", P, P, ref(good), 0, 0, 4096, None) == 0  # nothing to do
    assert _rc("ikv_append_paged_f32", P, P, ref(good), -1, 1, 4096, None) == -errno.EINVAL
    assert _rc("ikv_append_paged_f32", P, P, ref(good), 0, 1, 4100, None) == -errno.EINVAL
    assert _rc("ikv_append_paged_f32", P, P, None, 0, 1, 4096, None) == -errno.EINVAL
