"""GGUF files the reader tests share with tests/golden/make_gguf_golden.py.

Three families, each keyed by name:
  OPEN_CASES    a small container with metadata of every value type and
                tensors of several ggml types, valid and broken one field at a
                time (the malformations of the reference's own reader test,
                third_party/ingot/tests/test_gguf.c:304-410, and more);
  CONFIG_CASES  a one-layer Qwen3-shaped file whose metadata is varied the ways
                src/model.c:71-125 (load_config) and :177-228 (tensor binding)
                tell apart;
  SPLIT_CASES   split checkpoints (files and the name to open), read by
                ingot_gguf_open_split (gguf.h:62-66, gguf.c:466-570).
The golden script records, per case, whether the compiled reference's reader
(ingot_gguf_open) and loader (mynah_slm_load) accept it and which config it
reads; the tests hold this repository's reader to the same answers.
"""
from __future__ import annotations

import struct

import numpy as np

import gguf_writer as GW
from gguf_writer import (KV_ARRAY, KV_BOOL, KV_F32, KV_F64, KV_I8, KV_I16, KV_I32, KV_I64,
                         KV_STRING, KV_U8, KV_U16, KV_U32, KV_U64)


def _payload(ggml_type: int, ne, seed: int) -> bytes:
    n = GW.tensor_bytes(ggml_type, ne)
    raw = np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)
    if ggml_type == 0:                      # finite F32 values
        raw = np.random.default_rng(seed).standard_normal(n // 4).astype(np.float32).view(np.uint8)
    return raw.tobytes()


def mini_writer(version: int = 3, alignment: int = 32, append_alignment: bool = True):
    w = GW.GgufWriter(version=version, alignment=alignment, append_alignment=append_alignment)
    w.kv("general.architecture", KV_STRING, "mini")
    w.kv("mini.u8", KV_U8, 200).kv("mini.i8", KV_I8, -3).kv("mini.u16", KV_U16, 60000)
    w.kv("mini.i16", KV_I16, -20000).kv("mini.u32", KV_U32, 4000000000)
    w.kv("mini.i32", KV_I32, -100000).kv("mini.f32", KV_F32, 0.5).kv("mini.bool", KV_BOOL, 1)
    w.kv("mini.u64", KV_U64, 1 << 40).kv("mini.i64", KV_I64, -(1 << 40))
    w.kv("mini.f64", KV_F64, 2.75e9).kv("mini.big_f32", KV_F32, 3.0e38)
    w.kv("mini.neg_f64", KV_F64, -7.5)
    w.kv("mini.tokens", KV_ARRAY, ["a", "bb", "", "dddd"], KV_STRING)
    w.kv("mini.scores", KV_ARRAY, [1.5, -2.5, 0.25], KV_F32)
    w.kv("mini.empty", KV_ARRAY, [], KV_I32)
    for i, (name, t, ne) in enumerate((("f32.weight", 0, [8, 4]), ("f16.weight", 1, [16]),
                                       ("q8_0.weight", 8, [64, 2]), ("q4_k.weight", 12, [256, 3]),
                                       ("bf16.cube", 30, [4, 2, 3]), ("q6_k.weight", 14, [512]),
                                       ("q5_k.weight", 13, [256, 1]))):
        w.tensor(name, t, ne, _payload(t, ne, 100 + i))
    return w


def _patch(b: bytes, at: int, fmt: str, value) -> bytes:
    out = bytearray(b)
    struct.pack_into(fmt, out, at, value)
    return bytes(out)


def _mini(**kw):
    w = mini_writer(**kw)
    return w, w.to_bytes()


def _kv_value_at(w, key):
    return w.pos[("kv", key)]


def _open_cases():
    cases = {}
    w, b = _mini()
    last = w.tensors[-1]
    last_end = w.pos[("data", last[0])] + len(last[3])

    cases["valid_v3"] = lambda: b
    cases["valid_v2"] = lambda: _mini(version=2)[1]
    cases["no_alignment_key"] = lambda: _mini(append_alignment=False)[1]
    cases["alignment_16"] = lambda: _mini(alignment=16)[1]
    cases["alignment_64"] = lambda: _mini(alignment=64)[1]
    cases["trailing_padding_dropped"] = lambda: b[:last_end]
    cases["bad_magic"] = lambda: b"X" + b[1:]
    cases["version_1"] = lambda: _patch(b, 4, "<I", 1)
    cases["version_4"] = lambda: _patch(b, 4, "<I", 4)
    cases["version_9"] = lambda: _patch(b, 4, "<I", 9)
    cases["empty_file"] = lambda: b""
    cases["23_bytes"] = lambda: b[:23]
    cases["header_only"] = lambda: b[:24]
    cases["truncated_40"] = lambda: b[:40]
    cases["truncated_in_string_array"] = lambda: b[:_kv_value_at(w, "mini.tokens") + 20]
    cases["truncated_in_tensor_table"] = lambda: b[:w.pos[("ne", "q4_k.weight")] + 4]
    cases["truncated_before_data"] = lambda: b[:w.pos["data"] - 1]
    cases["last_payload_short"] = lambda: b[:last_end - 1]
    al = _kv_value_at(w, "general.alignment")
    for v in (0, 1, 8, 33, 48, 1 << 20, 1 << 21):
        cases[f"alignment_value_{v}"] = (lambda v=v: _patch(b, al, "<I", v))
    cases["alignment_as_u8"] = lambda: _patch(_patch(b, al - 4, "<I", KV_U8), al, "<I", 64)
    cases["huge_key_length"] = lambda: _patch(b, 24, "<Q", 0xFFFFFFFF)
    cases["key_length_16mib_plus_1"] = lambda: _patch(b, 24, "<Q", (16 << 20) + 1)
    sv = _kv_value_at(w, "general.architecture")
    cases["huge_string_value"] = lambda: _patch(b, sv, "<Q", 1 << 40)
    cases["bad_kv_type"] = lambda: _patch(b, sv - 4, "<I", 13)
    tok = _kv_value_at(w, "mini.tokens")
    cases["nested_array"] = lambda: _patch(b, tok, "<I", KV_ARRAY)
    cases["bad_array_type"] = lambda: _patch(b, tok, "<I", 13)
    cases["array_count_2pow28_plus_1"] = lambda: _patch(b, tok + 4, "<Q", (1 << 28) + 1)
    sc = _kv_value_at(w, "mini.scores")
    cases["array_count_past_file"] = lambda: _patch(b, sc + 4, "<Q", 1 << 27)
    cases["tensor_count_max"] = lambda: _patch(b, 8, "<Q", (1 << 64) - 1)
    cases["tensor_count_plus_one"] = lambda: _patch(b, 8, "<Q", len(w.tensors) + 1)
    cases["tensor_count_2pow28_plus_1"] = lambda: _patch(b, 8, "<Q", (1 << 28) + 1)
    cases["kv_count_max"] = lambda: _patch(b, 16, "<Q", (1 << 64) - 1)
    cases["kv_count_2pow28"] = lambda: _patch(b, 16, "<Q", 1 << 28)
    cases["kv_count_minus_one"] = lambda: _patch(b, 16, "<Q", len(w.kvs))
    for t in (4, 5, 31, 36, 42, 99):
        cases[f"tensor_type_{t}"] = (lambda t=t: _patch(b, w.pos[("type", "q6_k.weight")], "<I", t))
    cases["q4_k_as_q1_0"] = lambda: _patch(b, w.pos[("type", "q4_k.weight")], "<I", 41)
    cases["q8_0_as_q8_1"] = lambda: _patch(b, w.pos[("type", "q8_0.weight")], "<I", 9)
    cases["f16_as_nvfp4"] = lambda: _patch(b, w.pos[("type", "f16.weight")], "<I", 40)
    ne = w.pos[("ne", "q4_k.weight")]
    cases["zero_dimension"] = lambda: _patch(b, ne + 8, "<Q", 0)
    cases["zero_fast_dimension"] = lambda: _patch(b, ne, "<Q", 0)
    cases["q4_k_partial_block"] = lambda: _patch(b, ne, "<Q", 128)
    cases["dimension_overflow"] = lambda: _patch(_patch(b, ne, "<Q", 1 << 40), ne + 8, "<Q",
                                                 1 << 40)
    rk = w.pos[("ne", "f32.weight")] - 4
    cases["rank_9"] = lambda: _patch(b, rk, "<I", 9)
    cases["rank_0_f32"] = lambda: _patch(b, rk, "<I", 0)
    off = w.pos[("offset", "f32.weight")]
    cases["offset_unaligned"] = lambda: _patch(b, off, "<Q", 8)
    cases["offset_past_eof"] = lambda: _patch(b, off, "<Q", 1 << 20)
    cases["offset_wraps"] = lambda: _patch(b, off, "<Q", (1 << 64) - 32)
    lo = w.pos[("offset", last[0])]
    cases["last_offset_one_block_late"] = lambda: _patch(
        b, lo, "<Q", struct.unpack_from("<Q", b, lo)[0] + 32)

    def duplicate_name():
        d = mini_writer()
        d.tensors.append(("f16.weight",) + tuple(d.tensors[0][1:]))
        return d.to_bytes()

    cases["duplicate_tensor_name"] = duplicate_name
    return cases


# ── Qwen3 configs ──────────────────────────────────────────────────────────

QWEN3_KEYS = (("block_count", KV_U32, 1), ("embedding_length", KV_U32, 256),
              ("feed_forward_length", KV_U32, 512), ("attention.head_count", KV_U32, 4),
              ("attention.head_count_kv", KV_U32, 2), ("attention.key_length", KV_U32, 128),
              ("attention.value_length", KV_U32, 128), ("context_length", KV_U32, 40960),
              ("attention.layer_norm_rms_epsilon", KV_F32, 1e-6),
              ("rope.freq_base", KV_F32, 1000000.0))
LAYER_TENSORS = ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm", "ffn_gate",
                 "ffn_up", "ffn_down", "attn_q_norm", "attn_k_norm")


def config_writer(arch: str = "qwen3", keys=None, drop=(), tensors_drop=(), vocab: int = 64,
                  extra=(), embed_ne=None):
    """A one-layer file the reference loader binds: its metadata, and every
    tensor it looks up as a small F32 stand-in (the loader checks names, not
    shapes)."""
    w = GW.GgufWriter()
    if arch is not None:
        w.kv("general.architecture", KV_STRING, arch)
    for suffix, t, v in (keys if keys is not None else QWEN3_KEYS):
        if suffix not in drop:
            w.kv(f"{arch}.{suffix}", t, v)
    for key, t, v, at in extra:
        w.kv(key, t, v, at)
    names = ["token_embd.weight", "output_norm.weight"] + \
            [f"blk.0.{n}.weight" for n in LAYER_TENSORS]
    for i, n in enumerate(names):
        if n in tensors_drop:
            continue
        ne = (embed_ne or [8, vocab]) if n == "token_embd.weight" else [8]
        w.tensor(n, 0, ne, _payload(0, ne, 500 + i))
    return w


def _with(suffix, t, v):
    return tuple((s, t, v) if s == suffix else (s, tt, vv) for s, tt, vv in QWEN3_KEYS)


def _config_cases():
    c = {}
    c["qwen3_valid"] = lambda: config_writer().to_bytes()
    for suffix, _, _ in QWEN3_KEYS:
        if suffix != "attention.value_length":
            c[f"missing_{suffix}"] = (lambda s=suffix: config_writer(drop=(s,)).to_bytes())
    c["no_value_length"] = lambda: config_writer(drop=("attention.value_length",)).to_bytes()
    c["value_length_64"] = lambda: config_writer(
        keys=_with("attention.value_length", KV_U32, 64)).to_bytes()
    c["value_length_string"] = lambda: config_writer(
        keys=_with("attention.value_length", KV_STRING, "64")).to_bytes()
    c["value_length_f32_128"] = lambda: config_writer(
        keys=_with("attention.value_length", KV_F32, 128.0)).to_bytes()
    c["heads_not_multiple"] = lambda: config_writer(
        keys=_with("attention.head_count_kv", KV_U32, 3)).to_bytes()
    c["kv_heads_zero"] = lambda: config_writer(
        keys=_with("attention.head_count_kv", KV_U32, 0)).to_bytes()
    c["heads_zero"] = lambda: config_writer(
        keys=_with("attention.head_count", KV_U32, 0)).to_bytes()
    c["block_count_f32"] = lambda: config_writer(keys=_with("block_count", KV_F32, 1.0)).to_bytes()
    c["block_count_u64_truncates"] = lambda: config_writer(
        keys=_with("block_count", KV_U64, (1 << 32) + 1)).to_bytes()
    c["block_count_string"] = lambda: config_writer(
        keys=_with("block_count", KV_STRING, "1")).to_bytes()
    c["context_length_i64"] = lambda: config_writer(
        keys=_with("context_length", KV_I64, 2048)).to_bytes()
    c["rope_base_u32"] = lambda: config_writer(
        keys=_with("rope.freq_base", KV_U32, 10000)).to_bytes()
    c["eps_f64"] = lambda: config_writer(
        keys=_with("attention.layer_norm_rms_epsilon", KV_F64, 1e-5)).to_bytes()
    c["eps_string"] = lambda: config_writer(
        keys=_with("attention.layer_norm_rms_epsilon", KV_STRING, "1e-6")).to_bytes()
    c["no_architecture"] = lambda: config_writer(arch=None).to_bytes()
    c["empty_architecture"] = lambda: config_writer(arch="").to_bytes()
    c["arch_31_chars"] = lambda: config_writer(arch="q" * 31).to_bytes()
    c["arch_32_chars"] = lambda: config_writer(arch="q" * 32).to_bytes()
    c["other_arch_prefix"] = lambda: config_writer(arch="llama").to_bytes()
    c["duplicate_block_count"] = lambda: config_writer(
        extra=(("qwen3.block_count", KV_U32, 7, None),)).to_bytes()
    c["tokenizer_longer_than_embedding"] = lambda: config_writer(
        extra=(("tokenizer.ggml.tokens", KV_ARRAY, ["t"] * 70, KV_STRING),)).to_bytes()
    c["embedding_rank_1"] = lambda: config_writer(
        embed_ne=[8],
        extra=(("tokenizer.ggml.tokens", KV_ARRAY, ["t"] * 70, KV_STRING),)).to_bytes()
    c["missing_token_embd"] = lambda: config_writer(
        tensors_drop=("token_embd.weight",)).to_bytes()
    return c


OPEN_CASES = _open_cases()
CONFIG_CASES = _config_cases()
CONFIG_FIELDS = ("n_layers", "d_model", "d_ff", "n_heads", "n_kv_heads", "head_dim", "n_ctx",
                 "vocab", "rms_eps", "rope_theta")


# ── split checkpoints ──────────────────────────────────────────────────────

def _split_files(w, n=3, prefix="m", later_kvs=(), alignments=None):
    shards = GW.split_writers(w, n, later_kvs, alignments)
    return [[GW.split_name(prefix, i, n), s.to_bytes()] for i, s in enumerate(shards)], shards


def _split_cases():
    """name -> () -> (files [[file name, bytes]], the name to open): split
    checkpoints (<prefix>-0000k-of-0000n.gguf, gguf.h:62-66) whole and
    broken one shard at a time."""
    cases = {}
    later = (("general.architecture", KV_STRING, "mini", None),)

    def three():
        return _split_files(mini_writer(), 3, later_kvs=later)[0]

    cases["three_shards"] = lambda: (three(), GW.split_name("m", 0, 3))
    cases["open_via_second"] = lambda: (three(), GW.split_name("m", 1, 3))
    cases["open_via_last"] = lambda: (three(), GW.split_name("m", 2, 3))
    cases["two_shards_v2"] = lambda: (_split_files(mini_writer(version=2), 2)[0],
                                      GW.split_name("m", 0, 2))
    cases["later_alignment_64"] = lambda: (
        _split_files(mini_writer(), 3, alignments=[32, 64, 16])[0], GW.split_name("m", 0, 3))

    def later_align(value):
        files, shards = _split_files(mini_writer(), 3)
        b = shards[1].to_bytes()
        files[1][1] = _patch(b, shards[1].pos[("kv", "general.alignment")], "<I", value)
        return files

    cases["later_alignment_0"] = lambda: (later_align(0), GW.split_name("m", 0, 3))
    cases["later_alignment_48"] = lambda: (later_align(48), GW.split_name("m", 0, 3))

    def later_no_alignment_key():
        w = mini_writer()
        shards = GW.split_writers(w, 3)
        shards[2].append_alignment = False
        return [[GW.split_name("m", i, 3), s.to_bytes()] for i, s in enumerate(shards)]

    cases["later_no_alignment_key"] = lambda: (later_no_alignment_key(), GW.split_name("m", 0, 3))
    cases["missing_shard"] = lambda: (three()[:2], GW.split_name("m", 0, 3))

    def duplicate_across():
        w = mini_writer()
        shards = GW.split_writers(w, 3)
        shards[2].tensors.append(shards[0].tensors[0])
        return [[GW.split_name("m", i, 3), s.to_bytes()] for i, s in enumerate(shards)]

    cases["duplicate_across_shards"] = lambda: (duplicate_across(), GW.split_name("m", 0, 3))

    def broken_later(patch):
        files, shards = _split_files(mini_writer(), 3)
        files[2][1] = patch(shards[2], files[2][1])
        return files

    cases["later_bad_kv_type"] = lambda: (broken_later(
        lambda s, b: _patch(b, s.pos[("kv", "split.no")] - 4, "<I", 13)),
        GW.split_name("m", 0, 3))
    cases["later_version_1"] = lambda: (broken_later(lambda s, b: _patch(b, 4, "<I", 1)),
                                        GW.split_name("m", 0, 3))
    cases["later_truncated"] = lambda: (broken_later(lambda s, b: b[:s.pos["data"] - 1]),
                                        GW.split_name("m", 0, 3))
    cases["later_payload_past_eof"] = lambda: (broken_later(
        lambda s, b: _patch(b, s.pos[("offset", s.tensors[-1][0])], "<Q", 1 << 20)),
        GW.split_name("m", 0, 3))
    cases["one_of_one_is_plain"] = lambda: ([[GW.split_name("m", 0, 1), mini_writer().to_bytes()]],
                                            GW.split_name("m", 0, 1))
    cases["number_past_total_is_plain"] = lambda: (
        [["m-00004-of-00003.gguf", mini_writer().to_bytes()]], "m-00004-of-00003.gguf")
    cases["plain_name"] = lambda: ([["m.gguf", mini_writer().to_bytes()]], "m.gguf")
    return cases


SPLIT_CASES = _split_cases()
