"""GGUF v3 files for the Qwen3 models: a writer of the benchmark
configurations' synthetic weights and a reader that feeds a GGUF F32 model to
``Qwen3Engine``.

The file layout is the public GGUF v3 format the reference parses
(src/gguf_parser.cpp:100-284): magic "GGUF", version 3, tensor and metadata
counts, metadata key/value pairs, tensor infos (name, dims innermost first,
type, offset), padding to ``general.alignment`` (32 when absent), tensor data.
The keys written are those ModelBase::load_hparams reads
(src/model.cpp:60-163) and the tensor names those ModelBase::load_weight
reads (src/model.cpp:164-311). ``output.weight`` is written only for a
config with ``untied_output``; without it the logits use the tied token
embedding, and a file that has one is read as untied (src/model.cpp:203-210).
A file written here therefore runs on the reference's CPU backend as well,
e.g. for its config-0 benchmark.

    python -m ikv.gguf write --config 0 --out qwen3-0.6b-synthetic.gguf

Only F32 tensors are read or written.
"""
from __future__ import annotations

import argparse
import dataclasses
import struct
from typing import BinaryIO, Dict, Iterable, Optional, Tuple

import numpy as np

MAGIC = 0x46554747  # "GGUF", little endian
VERSION = 3
ALIGNMENT = 32

# metadata value types
T_UINT8, T_INT8, T_UINT16, T_INT16, T_UINT32, T_INT32, T_FLOAT32, T_BOOL, T_STRING, T_ARRAY, \
    T_UINT64, T_INT64, T_FLOAT64 = range(13)
_SCALAR = {T_UINT8: "<B", T_INT8: "<b", T_UINT16: "<H", T_INT16: "<h", T_UINT32: "<I",
           T_INT32: "<i", T_FLOAT32: "<f", T_BOOL: "<?", T_UINT64: "<Q", T_INT64: "<q",
           T_FLOAT64: "<d"}
GGML_TYPE_F32 = 0


# ---------------------------------------------------------------------------
# writing
# ---------------------------------------------------------------------------

def _w_str(f: BinaryIO, s: str) -> None:
    b = s.encode("utf-8")
    f.write(struct.pack("<Q", len(b)))
    f.write(b)


def _w_value(f: BinaryIO, vtype: int, value) -> None:
    if vtype == T_STRING:
        _w_str(f, value)
    elif vtype == T_ARRAY:
        etype, items = value
        f.write(struct.pack("<IQ", etype, len(items)))
        for it in items:
            _w_value(f, etype, it)
    else:
        f.write(struct.pack(_SCALAR[vtype], value))


def qwen3_metadata(cfg, name: str = "qwen3-synthetic", tokens: Optional[Iterable[str]] = None):
    """(key, type, value) of the hyperparameters ModelBase::load_hparams
    reads (src/model.cpp:60-163) for a Qwen3 config."""
    toks = list(tokens) if tokens is not None else [f"<t{i}>" for i in range(cfg.n_vocab)]
    if len(toks) != cfg.n_vocab:
        raise ValueError("one token string per vocabulary entry")
    p = "qwen3."
    return [
        ("general.architecture", T_STRING, "qwen3"),
        ("general.name", T_STRING, name),
        ("general.alignment", T_UINT32, ALIGNMENT),
        (p + "embedding_length", T_UINT32, cfg.n_embd),
        (p + "block_count", T_UINT32, cfg.n_layer),
        (p + "attention.head_count", T_UINT32, cfg.n_head),
        (p + "attention.head_count_kv", T_UINT32, cfg.n_head_kv),
        (p + "feed_forward_length", T_UINT32, cfg.n_ff),
        (p + "context_length", T_UINT32, cfg.n_ctx_train),
        (p + "attention.key_length", T_UINT32, cfg.head_dim),
        (p + "attention.value_length", T_UINT32, cfg.head_dim),
        (p + "rope.freq_base", T_FLOAT32, float(cfg.rope_theta)),
        (p + "attention.layer_norm_rms_epsilon", T_FLOAT32, float(cfg.rms_norm_eps)),
        ("tokenizer.ggml.tokens", T_ARRAY, (T_STRING, toks)),
    ]


def write(path, metadata, tensors) -> None:
    """GGUF v3 file of `metadata` ((key, type, value) triples) and `tensors`
    ((name, shape row-major, source) triples; source is an array or a
    callable(i0, i1) -> float32 values of flat elements [i0, i1), so large
    tensors stream to disk)."""
    tensors = list(tensors)
    with open(path, "wb") as f:
        f.write(struct.pack("<IIQQ", MAGIC, VERSION, len(tensors), len(metadata)))
        for key, vtype, value in metadata:
            _w_str(f, key)
            f.write(struct.pack("<I", vtype))
            _w_value(f, vtype, value)
        offset = 0
        for name, shape, _ in tensors:
            _w_str(f, name)
            ne = list(reversed(shape))  # dims innermost first
            f.write(struct.pack("<I", len(ne)))
            f.write(struct.pack(f"<{len(ne)}Q", *ne))
            f.write(struct.pack("<IQ", GGML_TYPE_F32, offset))
            offset += -(-int(np.prod(shape)) * 4 // ALIGNMENT) * ALIGNMENT
        f.write(b"\0" * (-f.tell() % ALIGNMENT))
        for name, shape, src in tensors:
            n = int(np.prod(shape))
            if callable(src):
                chunk = 1 << 24
                for i0 in range(0, n, chunk):
                    f.write(np.ascontiguousarray(src(i0, min(n, i0 + chunk)), np.float32).tobytes())
            else:
                a = np.ascontiguousarray(src, np.float32)
                if a.size != n:
                    raise ValueError(f"{name}: {a.size} values for shape {shape}")
                f.write(a.tobytes())
            f.write(b"\0" * (-(n * 4) % ALIGNMENT))


def write_qwen3_synthetic(path, cfg, seed: int, std: float = 0.02, name: str = "qwen3-synthetic",
                          threads: int = 8) -> None:
    """The benchmark configurations' random-init model (ikv_qwen3_init_synthetic's
    weights, bit for bit: one N(0, std^2) stream in tensor order, norms 1.0)."""
    from . import qwen3, synth_normal

    offset = 0
    tensors = []
    for tname, shape in qwen3.tensor_layout(cfg):
        n = int(np.prod(shape))
        if "norm" in tname:
            tensors.append((tname, shape, np.ones(n, np.float32)))
            continue

        def src(i0, i1, base=offset):
            return synth_normal(seed, (i1 - i0,), std=std, offset=base + i0, threads=threads)
        tensors.append((tname, shape, src))
        offset += n
    write(path, qwen3_metadata(cfg, name), tensors)


# ---------------------------------------------------------------------------
# reading
# ---------------------------------------------------------------------------

@dataclasses.dataclass
class TensorInfo:
    name: str
    shape: Tuple[int, ...]  # row-major (outermost first)
    ggml_type: int
    offset: int             # from the start of the data region


def _r(f: BinaryIO, fmt: str):
    size = struct.calcsize(fmt)
    b = f.read(size)
    if len(b) != size:
        raise ValueError("truncated GGUF file")
    return struct.unpack(fmt, b)


def _r_str(f: BinaryIO) -> str:
    (n,) = _r(f, "<Q")
    b = f.read(n)
    if len(b) != n:
        raise ValueError("truncated GGUF string")
    return b.decode("utf-8")


def _r_value(f: BinaryIO, vtype: int):
    if vtype == T_STRING:
        return _r_str(f)
    if vtype == T_ARRAY:
        etype, n = _r(f, "<IQ")
        return [_r_value(f, etype) for _ in range(n)]
    if vtype not in _SCALAR:
        raise ValueError(f"unknown GGUF value type {vtype}")
    return _r(f, _SCALAR[vtype])[0]


class GGUFFile:
    """Metadata and F32 tensors of a GGUF v3 file; tensors are memory-mapped."""

    def __init__(self, path):
        self.path = str(path)
        with open(self.path, "rb") as f:
            magic, version, n_tensors, n_kv = _r(f, "<IIQQ")
            if magic != MAGIC:
                raise ValueError("not a GGUF file")
            if version != VERSION:
                raise ValueError(f"GGUF version {version}; only 3 is read")
            self.metadata: Dict[str, object] = {}
            for _ in range(n_kv):
                key = _r_str(f)
                (vtype,) = _r(f, "<I")
                self.metadata[key] = _r_value(f, vtype)
            self.tensors: Dict[str, TensorInfo] = {}
            for _ in range(n_tensors):
                name = _r_str(f)
                (nd,) = _r(f, "<I")
                ne = _r(f, f"<{nd}Q")
                gtype, off = _r(f, "<IQ")
                self.tensors[name] = TensorInfo(name, tuple(reversed(ne)), gtype, off)
            align = int(self.metadata.get("general.alignment", ALIGNMENT))
            self.data_offset = -(-f.tell() // align) * align
        self._map = np.memmap(self.path, dtype=np.uint8, mode="r")

    def tensor(self, name: str) -> np.ndarray:
        info = self.tensors[name]
        if info.ggml_type != GGML_TYPE_F32:
            raise ValueError(f"{name}: GGML type {info.ggml_type}; only F32 is read")
        n = int(np.prod(info.shape))
        start = self.data_offset + info.offset
        if start + 4 * n > self._map.size:
            raise ValueError(f"{name}: data past the end of the file")
        return self._map[start:start + 4 * n].view(np.float32).reshape(info.shape)


def qwen3_config(g: GGUFFile):
    """Qwen3Config from the keys of src/model.cpp:60-163 (with its defaults)."""
    from . import qwen3

    m = g.metadata
    arch = m["general.architecture"]
    p = f"{arch}."
    n_embd, n_head = int(m[p + "embedding_length"]), int(m[p + "attention.head_count"])
    return qwen3.Qwen3Config(
        n_layer=int(m[p + "block_count"]), n_embd=n_embd, n_head=n_head,
        n_head_kv=int(m[p + "attention.head_count_kv"]),
        head_dim=int(m.get(p + "attention.key_length", n_embd // n_head)),
        n_ff=int(m[p + "feed_forward_length"]), n_vocab=len(m["tokenizer.ggml.tokens"]),
        n_ctx_train=int(m[p + "context_length"]),
        rope_theta=float(m.get(p + "rope.freq_base", 10000.0)),
        rms_norm_eps=float(m.get(p + "attention.layer_norm_rms_epsilon", 1e-5)),
        untied_output=int("output.weight" in g.tensors))


def load_qwen3(path, max_ctx: int, device: int = 0, **engine_kw):
    """A Qwen3Engine with the weights of a GGUF F32 Qwen3 model file."""
    from . import qwen3

    g = GGUFFile(path)
    cfg = qwen3_config(g)
    eng = qwen3.Qwen3Engine(cfg, max_ctx, device=device, **engine_kw)
    eng.set_weights({name: g.tensor(name) for name, _ in qwen3.tensor_layout(cfg)})
    return eng


def main(argv=None) -> None:
    from . import qwen3, synth

    ap = argparse.ArgumentParser(prog="python -m ikv.gguf")
    sub = ap.add_subparsers(dest="cmd", required=True)
    w = sub.add_parser("write", help="the synthetic model of a benchmark configuration")
    w.add_argument("--config", type=int, default=0, choices=(0, 3, 4))
    w.add_argument("--out", required=True)
    w.add_argument("--threads", type=int, default=8)
    args = ap.parse_args(argv)
    arch = {0: qwen3.QWEN3_0_6B, 3: qwen3.QWEN3_0_6B, 4: qwen3.QWEN3_8B}[args.config]
    write_qwen3_synthetic(args.out, arch, synth.config_seed(args.config, 1), threads=args.threads,
                          name=f"qwen3-synthetic-config{args.config}")


if __name__ == "__main__":
    main()
