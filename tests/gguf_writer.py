"""GGUF v2 / v3 files for the tests (test infrastructure only).

Writes the container the way the reference's writer lays it out
(third_party/ingot/src/write.c:259-330, ingot_gguf_writer_save): header
(magic "GGUF", version 3, tensor count, metadata count), the metadata in
insertion order with general.alignment = 32 (u32) appended last, the tensor
table (name, rank, ne[0..rank), ggml type, offset), zero padding to 32, then
each payload followed by zero padding to 32; offsets are the running sum of
the payload sizes rounded up to 32. The bytes of `qwen3_gguf` are pinned to
the reference writer's output for the same model (test_gguf.py: a live
comparison with the compiled reference where it is built, and the SHA-256
recorded in tests/golden/gguf_qwen3_tiny.json everywhere).

Every field's byte position is recorded in `GgufWriter.pos`, so the
malformed-file tests can patch one field and nothing else.
"""
from __future__ import annotations

import struct

MAGIC = 0x46554747
(KV_U8, KV_I8, KV_U16, KV_I16, KV_U32, KV_I32, KV_F32, KV_BOOL, KV_STRING, KV_ARRAY, KV_U64,
 KV_I64, KV_F64) = range(13)
_SCALAR = {KV_U8: "<B", KV_I8: "<b", KV_U16: "<H", KV_I16: "<h", KV_U32: "<I", KV_I32: "<i",
           KV_F32: "<f", KV_BOOL: "<B", KV_U64: "<Q", KV_I64: "<q", KV_F64: "<d"}

# (values, bytes) per block of the ggml types the tests write.
GEOMETRY = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144),
            13: (256, 176), 14: (256, 210)}


def _str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(kv_type: int, value, arr_type: int | None = None) -> bytes:
    if kv_type == KV_STRING:
        return _str(value)
    if kv_type == KV_ARRAY:
        body = b"".join(_value(arr_type, v) for v in value)
        return struct.pack("<IQ", arr_type, len(value)) + body
    return struct.pack(_SCALAR[kv_type], value)


def tensor_bytes(ggml_type: int, ne) -> int:
    elems, nbytes = GEOMETRY[ggml_type]
    n = 1
    for d in ne:
        n *= d
    return n // elems * nbytes


class GgufWriter:
    def __init__(self, version: int = 3, alignment: int = 32, append_alignment: bool = True):
        self.version, self.alignment = version, alignment
        self.append_alignment = append_alignment
        self.kvs: list[tuple[str, int, object, int | None]] = []
        self.tensors: list[tuple[str, int, list, bytes]] = []
        self.pos: dict = {}

    def kv(self, key: str, kv_type: int, value, arr_type: int | None = None) -> "GgufWriter":
        self.kvs.append((key, kv_type, value, arr_type))
        return self

    def tensor(self, name: str, ggml_type: int, ne, data: bytes) -> "GgufWriter":
        self.tensors.append((name, ggml_type, list(ne), bytes(data)))
        return self

    def to_bytes(self) -> bytes:
        a = self.alignment
        kvs = list(self.kvs)
        if self.append_alignment:
            kvs.append(("general.alignment", KV_U32, a, None))
        out = bytearray(struct.pack("<IIQQ", MAGIC, self.version, len(self.tensors), len(kvs)))
        for key, t, v, at in kvs:
            out += _str(key) + struct.pack("<I", t)
            self.pos.setdefault(("kv", key), len(out))
            out += _value(t, v, at)
        offset = 0
        for name, t, ne, data in self.tensors:
            self.pos[("tensor", name)] = len(out)
            out += _str(name) + struct.pack("<I", len(ne))
            self.pos[("ne", name)] = len(out)
            out += b"".join(struct.pack("<Q", d) for d in ne)
            self.pos[("type", name)] = len(out)
            out += struct.pack("<I", t)
            self.pos[("offset", name)] = len(out)
            out += struct.pack("<Q", offset)
            offset += (len(data) + a - 1) // a * a
        out += bytes(-len(out) % a)
        self.pos["data"] = len(out)
        for name, _, _, data in self.tensors:
            self.pos[("data", name)] = len(out)
            out += data + bytes(-len(data) % a)
        return bytes(out)


def qwen3_writer(shape, table, count: int, blob, n_ctx: int) -> GgufWriter:
    """A random-init Qwen3 as a GGUF, in the key and tensor order
    oracle/ref_harness.c (ref_write_qwen3_gguf) hands the reference writer."""
    w = GgufWriter()
    w.kv("general.architecture", KV_STRING, "qwen3")
    for key, val in (("block_count", shape.n_layers), ("embedding_length", shape.d_model),
                     ("feed_forward_length", shape.d_ff),
                     ("attention.head_count", shape.n_heads),
                     ("attention.head_count_kv", shape.n_kv_heads),
                     ("attention.key_length", shape.head_dim),
                     ("attention.value_length", shape.head_dim), ("context_length", n_ctx)):
        w.kv("qwen3." + key, KV_U32, val)
    w.kv("qwen3.attention.layer_norm_rms_epsilon", KV_F32, shape.rms_eps)
    w.kv("qwen3.rope.freq_base", KV_F32, shape.rope_theta)
    raw = memoryview(blob).cast("B")
    for i in range(count):
        t = table[i]
        ne = [t.cols] if t.rank == 1 else [t.cols, t.rows]
        w.tensor(t.name.decode(), t.type, ne, raw[t.offset:t.offset + t.nbytes])
    return w


def qwen3_gguf(shape, table, count: int, blob, n_ctx: int) -> bytes:
    return qwen3_writer(shape, table, count, blob, n_ctx).to_bytes()


def split_writers(w: GgufWriter, n: int, later_kvs=(), alignments=None) -> list:
    """w's tensors spread over n shards, a contiguous run each, in order (as
    llama.cpp's gguf-split writes them): shard 0 carries w's metadata, later
    shards only `later_kvs`;
    every shard also gets split.no / split.count / split.tensors.count
    (u16, u16, i32) like gguf-split's. alignments[i] sets shard i's."""
    per = -(-len(w.tensors) // n)
    out = []
    for i in range(n):
        a = alignments[i] if alignments else w.alignment
        s = GgufWriter(version=w.version, alignment=a, append_alignment=w.append_alignment)
        if i == 0:
            s.kvs = list(w.kvs)
        else:
            s.kvs = list(later_kvs)
        s.kv("split.no", KV_U16, i).kv("split.count", KV_U16, n)
        s.kv("split.tensors.count", KV_I32, len(w.tensors))
        s.tensors = w.tensors[i * per:(i + 1) * per]
        out.append(s)
    return out


def split_name(prefix: str, i: int, n: int) -> str:
    return f"{prefix}-{i + 1:05d}-of-{n:05d}.gguf"
