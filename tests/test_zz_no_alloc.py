"""ikv_attn_decode_noalloc_f32, the decode entry point that allocates nothing:
called through the C-ABI, its output and cache rows must be bit-identical to
ikv_attn_decode_f32's with a fresh workspace, on calls in a row that share the
library's device scratch array (the later ones smaller, and of another head
shape, so that partials a previous call left where this call's arrival
counters sit must be cleared)."""
import ctypes
import errno

import numpy as np
import pytest
import torch

import ikv

D = 128


def _noalloc(q, kc, vc, kn, vn, out, n_kv, scale=0.0):
    n_head, n_head_kv = q.shape[0], kc.shape[1]
    return ikv.load().ikv_attn_decode_noalloc_f32(
        ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(kc.data_ptr()),
        ctypes.c_void_p(vc.data_ptr()),
        None if kn is None else ctypes.c_void_p(kn.data_ptr()),
        None if vn is None else ctypes.c_void_p(vn.data_ptr()),
        ctypes.c_void_p(out.data_ptr()), n_head, n_head_kv, D, n_kv, scale,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def _case(dev, seed, n_head, n_head_kv, n_kv, fused):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rnd = lambda *s: torch.randn(s, generator=g, device=dev, dtype=torch.float32)  # noqa: E731
    kc, vc = rnd(n_kv + 3, n_head_kv, D), rnd(n_kv + 3, n_head_kv, D)
    q = rnd(n_head, D)
    kn, vn = (rnd(n_head_kv, D), rnd(n_head_kv, D)) if fused else (None, None)
    return q, kc, vc, kn, vn


def _bits(t):
    return t.cpu().numpy().view(np.uint32)


# (n_head, n_head_kv, n_kv, fused): the first call uses most of the array
# (64/8 heads at 40960 keys: 1.07 MB of partials); the next ones are smaller,
# of other head shapes, and one fits a single split (no scratch use at all)
CALLS = [(64, 8, 40960, True), (16, 8, 1500, True), (32, 4, 4097, False), (16, 8, 100, True)]


@pytest.mark.gpu
def test_noalloc_decode_equals_workspace_decode(dev):
    for i, (hq, hkv, n_kv, fused) in enumerate(CALLS):
        print(f"noalloc call {i}: n_head={hq} n_head_kv={hkv} n_kv={n_kv} fused={fused}", flush=True)
        assert ikv.decode_workspace_bytes(hq, hkv, D, n_kv) <= ikv.NOALLOC_SCRATCH_BYTES
        q, kc, vc, kn, vn = _case(dev, 100 + i, hq, hkv, n_kv, fused)
        kc2, vc2 = kc.clone(), vc.clone()
        out = torch.full((hq, D), float("nan"), device=dev)
        assert _noalloc(q, kc, vc, kn, vn, out, n_kv) == 0
        want = ikv.attn_decode(q, kc2, vc2, n_kv, k_new=kn, v_new=vn)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(out), _bits(want)), f"call {i}: output differs"
        assert np.array_equal(_bits(kc), _bits(kc2)), f"call {i}: K cache differs"
        assert np.array_equal(_bits(vc), _bits(vc2)), f"call {i}: V cache differs"


@pytest.mark.gpu
def test_noalloc_decode_repeats_bit_identically(dev):
    # the same call twice with a different-shape call between them
    q, kc, vc, _, _ = _case(dev, 7, 16, 8, 8200, False)
    a = torch.empty((16, D), device=dev)
    b = torch.empty((16, D), device=dev)
    assert _noalloc(q, kc, vc, None, None, a, 8200) == 0
    q2, kc2, vc2, _, _ = _case(dev, 8, 32, 8, 3000, False)
    mid = torch.empty((32, D), device=dev)
    assert _noalloc(q2, kc2, vc2, None, None, mid, 3000) == 0
    assert _noalloc(q, kc, vc, None, None, b, 8200) == 0
    torch.cuda.synchronize()
    assert np.array_equal(_bits(a), _bits(b))


@pytest.mark.gpu
def test_noalloc_decode_rejects_what_does_not_fit(dev):
    # 4096 query heads over 512 KV heads need 2.26 MB of partials; the
    # rejection comes before any launch or pointer use
    assert ikv.decode_workspace_bytes(4096, 512, D, 4097) > ikv.NOALLOC_SCRATCH_BYTES
    t = torch.zeros(64, device=dev)
    p = ctypes.c_void_p(t.data_ptr())
    rc = ikv.load().ikv_attn_decode_noalloc_f32(p, p, p, None, None, p, 4096, 512, D, 4097, 0.0,
                                                None)
    assert rc == -errno.ENOSPC
    # and a shape that does fit still runs after the rejection
    q, kc, vc, kn, vn = _case(dev, 9, 16, 8, 600, True)
    kc2, vc2 = kc.clone(), vc.clone()
    out = torch.empty((16, D), device=dev)
    assert _noalloc(q, kc, vc, kn, vn, out, 600) == 0
    want = ikv.attn_decode(q, kc2, vc2, 600, k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), _bits(want))


@pytest.mark.gpu
def test_noalloc_decode_replays_from_a_captured_graph(dev):
    # For callers under HIP graph capture: after a first call on the device
    # outside capture (which looks up the scratch array's address), one call
    # is captured and replayed; every replay equals the workspace form bit for
    # bit (output and the appended cache rows), with eager work in between.
    q, kc, vc, kn, vn = _case(dev, 21, 16, 8, 3000, True)
    kc2, vc2 = kc.clone(), vc.clone()
    want = ikv.attn_decode(q, kc2, vc2, 3000, k_new=kn, v_new=vn)
    out = torch.full((16, D), float("nan"), device=dev)
    assert _noalloc(q, kc, vc, kn, vn, out, 3000) == 0
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), _bits(want))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = _noalloc(q, kc, vc, kn, vn, out, 3000)
    assert rc == 0
    torch.cuda.current_stream().wait_stream(side)
    for i in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(out), _bits(want)), f"replay {i}: output differs"
        assert np.array_equal(_bits(kc), _bits(kc2)), f"replay {i}: K cache differs"
        assert np.array_equal(_bits(vc), _bits(vc2)), f"replay {i}: V cache differs"
