"""GGUF v3 writer and reader (infer-llm_amd/ikv/gguf.py) on the CPU: the
layout the reference parses (src/gguf_parser.cpp:100-284), the keys and
tensor names its loader reads (src/model.cpp:60-311), a bit-exact round trip
of the synthetic weights, and rejection of malformed files."""
import dataclasses
import struct

import numpy as np
import pytest

from ikv import gguf, qwen3

TINY = qwen3.Qwen3Config(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512,
                         n_vocab=300, n_ctx_train=1024)


@pytest.fixture(scope="module")
def tiny_file(tmp_path_factory):
    path = tmp_path_factory.mktemp("gguf") / "tiny.gguf"
    gguf.write_qwen3_synthetic(path, TINY, seed=1234, threads=2)
    return path


def test_header_and_alignment(tiny_file):
    raw = tiny_file.read_bytes()
    magic, version, n_t, n_kv = struct.unpack("<IIQQ", raw[:24])
    assert raw[:4] == b"GGUF" and magic == gguf.MAGIC and version == 3
    assert n_t == len(qwen3.tensor_layout(TINY)) and n_kv == 14
    g = gguf.GGUFFile(tiny_file)
    assert g.data_offset % 32 == 0
    assert all(t.offset % 32 == 0 for t in g.tensors.values())
    last = max(g.tensors.values(), key=lambda t: t.offset)
    assert g.data_offset + last.offset + 4 * int(np.prod(last.shape)) <= len(raw)


def test_keys_the_reference_loader_reads(tiny_file):
    g = gguf.GGUFFile(tiny_file)
    m = g.metadata
    assert m["general.architecture"] == "qwen3" and isinstance(m["general.name"], str)
    assert len(m["tokenizer.ggml.tokens"]) == TINY.n_vocab
    for key, want in [("embedding_length", 256), ("block_count", 2), ("attention.head_count", 4),
                      ("attention.head_count_kv", 2), ("feed_forward_length", 512),
                      ("context_length", 1024), ("attention.key_length", 64),
                      ("attention.value_length", 64)]:
        assert m["qwen3." + key] == want, key
    assert m["qwen3.rope.freq_base"] == np.float32(1e6)
    assert m["qwen3.attention.layer_norm_rms_epsilon"] == np.float32(1e-6)
    c = gguf.qwen3_config(g)  # the float keys are float32 in the file, as in the engine's ABI
    assert dataclasses.replace(c, rope_theta=TINY.rope_theta, rms_norm_eps=TINY.rms_norm_eps) == TINY
    assert np.float32(c.rms_norm_eps) == np.float32(TINY.rms_norm_eps)
    assert np.float32(c.rope_theta) == np.float32(TINY.rope_theta)
    # tied embedding: no output.weight; per-layer names of src/model.cpp:214-306
    assert "output.weight" not in g.tensors
    for name in ("token_embd.weight", "output_norm.weight", "blk.1.attn_q.weight",
                 "blk.1.attn_k_norm.weight", "blk.0.ffn_down.weight"):
        assert name in g.tensors
    # dims: GGUF ne = (k, n_out) for a [n_out][k] matrix
    assert g.tensors["blk.0.attn_q.weight"].shape == (4 * 64, 256)
    assert g.tensors["blk.0.ffn_down.weight"].shape == (256, 512)


def test_round_trip_is_bit_exact(tiny_file):
    g = gguf.GGUFFile(tiny_file)
    want = qwen3.synthetic_weights(TINY, 1234, threads=2)
    for name, arr in want.items():
        got = g.tensor(name)
        assert got.shape == arr.shape
        assert np.array_equal(got.view(np.uint32), arr.view(np.uint32)), name


def test_untied_output_round_trips(tmp_path):
    # a model with its own output projection (src/model.cpp:203-210): the
    # writer emits output.weight, the reader sees it and marks the config
    # untied, and the projection is drawn after every tied-model tensor, so
    # the shared tensors equal the tied model's bit for bit
    untied = dataclasses.replace(TINY, untied_output=1)
    path = tmp_path / "untied.gguf"
    gguf.write_qwen3_synthetic(path, untied, seed=1234, threads=2)
    g = gguf.GGUFFile(path)
    assert gguf.qwen3_config(g).untied_output == 1
    assert g.tensors["output.weight"].shape == (TINY.n_vocab, TINY.n_embd)
    assert [n for n, _ in qwen3.tensor_layout(untied)][-1] == "output.weight"
    want = qwen3.synthetic_weights(untied, 1234, threads=2)
    tied = qwen3.synthetic_weights(TINY, 1234, threads=2)
    assert set(want) == set(tied) | {"output.weight"}
    for name, arr in want.items():
        assert np.array_equal(g.tensor(name).view(np.uint32), arr.view(np.uint32)), name
        if name in tied:
            assert np.array_equal(arr, tied[name]), name
    assert not np.array_equal(want["output.weight"], want["token_embd.weight"])


def test_malformed_files_are_rejected(tmp_path, tiny_file):
    raw = bytearray(tiny_file.read_bytes())
    bad = tmp_path / "bad_magic.gguf"
    bad.write_bytes(b"GGUG" + bytes(raw[4:]))
    with pytest.raises(ValueError, match="not a GGUF"):
        gguf.GGUFFile(bad)
    v2 = tmp_path / "v2.gguf"
    v2.write_bytes(bytes(raw[:4]) + struct.pack("<I", 2) + bytes(raw[8:]))
    with pytest.raises(ValueError, match="version"):
        gguf.GGUFFile(v2)
    cut = tmp_path / "cut.gguf"
    cut.write_bytes(bytes(raw[:200]))
    with pytest.raises(ValueError, match="truncated"):
        gguf.GGUFFile(cut)
    # a tensor of another type is named, not misread
    f16 = tmp_path / "f16.gguf"
    gguf.write(f16, [("general.architecture", gguf.T_STRING, "x")],
               [("w", (2, 16), np.zeros(32, np.float32))])
    data = bytearray(f16.read_bytes())
    i = data.index(b"w") + 1 + 4 + 16           # name, n_dims, two dims
    data[i:i + 4] = struct.pack("<I", 1)        # GGML_TYPE_F16
    f16.write_bytes(bytes(data))
    with pytest.raises(ValueError, match="only F32"):
        gguf.GGUFFile(f16).tensor("w")


def test_metadata_value_types_round_trip(tmp_path):
    meta = [("a.u8", gguf.T_UINT8, 7), ("a.i32", gguf.T_INT32, -5), ("a.f64", gguf.T_FLOAT64, 0.1),
            ("a.bool", gguf.T_BOOL, True), ("a.u64", gguf.T_UINT64, 2**40),
            ("a.arr", gguf.T_ARRAY, (gguf.T_INT16, [1, -2, 3])),
            ("a.nested", gguf.T_ARRAY, (gguf.T_ARRAY, [(gguf.T_UINT8, [1]), (gguf.T_UINT8, [2, 3])]))]
    p = tmp_path / "m.gguf"
    gguf.write(p, meta, [])
    m = gguf.GGUFFile(p).metadata
    assert m["a.u8"] == 7 and m["a.i32"] == -5 and m["a.f64"] == 0.1 and m["a.bool"] is True
    assert m["a.u64"] == 2**40 and m["a.arr"] == [1, -2, 3] and m["a.nested"] == [[1], [2, 3]]
