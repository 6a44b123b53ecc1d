"""ctypes access to the CPU checkers under oracle/ (test infrastructure only).

  * liboracle.so    this repository's C11 restatement of the reference path
  * _ref/libref.so  the reference compiled from its own sources (built here
                    when /root/reference exists; optional everywhere else)
  * _ref/libref_int8.so  ingot's kernels built with AVX2 + FMA, the build in
                    which the reference's int8 activation lane exists
"""
from __future__ import annotations

import ctypes as C
import os
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libref.so")
REF_INT8_SO = os.path.join(ROOT, "oracle", "_ref", "libref_int8.so")

_P, _SZ = C.c_void_p, C.c_size_t


class OrcTensor(C.Structure):
    _fields_ = [("type", C.c_int), ("rows", C.c_uint64), ("cols", C.c_uint64), ("data", _P)]


class OrcLayer(C.Structure):
    _fields_ = [(n, OrcTensor) for n in ("attn_norm", "wq", "wk", "wv", "q_norm", "k_norm", "wo",
                                         "ffn_norm", "gate", "up", "down")]


class OrcConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("n_layers", "d_model", "d_ff", "n_heads", "n_kv_heads",
                                          "head_dim", "vocab")] + \
               [("rms_eps", C.c_float), ("rope_theta", C.c_float)]


class SynthShape(C.Structure):
    _fields_ = OrcConfig._fields_


class SynthTensor(C.Structure):
    _fields_ = [("name", C.c_char * 48), ("type", C.c_int), ("rank", C.c_uint32),
                ("rows", C.c_uint64), ("cols", C.c_uint64), ("offset", C.c_uint64),
                ("nbytes", C.c_uint64)]


class RefTensor(C.Structure):
    """ingot_tensor (third_party/ingot/include/ingot/gguf.h:41-50)."""
    _fields_ = [("name", C.c_char_p), ("type", C.c_int), ("rank", C.c_uint32),
                ("ne", C.c_uint64 * 8), ("nelem", C.c_uint64), ("nbytes", C.c_uint64),
                ("offset", C.c_uint64), ("shard", C.c_uint32)]


class SamplerParams(C.Structure):
    """mynah_slm_sampler_params (src/sampler.h:16-30) = orc_sampler_params."""
    _fields_ = [("temp", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float),
                ("min_p", C.c_float), ("repeat_penalty", C.c_float), ("freq_penalty", C.c_float),
                ("presence_penalty", C.c_float), ("penalty_window", C.c_uint32),
                ("seed", C.c_uint64)]


def sampler_params(temp=0.0, top_k=0, top_p=1.0, min_p=0.0, repeat_penalty=1.0,
                   freq_penalty=0.0, presence_penalty=0.0, penalty_window=64, seed=0):
    return SamplerParams(temp, top_k, top_p, min_p, repeat_penalty, freq_penalty,
                         presence_penalty, penalty_window, seed)


class RefConfig(C.Structure):
    """mynah_slm_config (src/model.h:25-48)."""
    _fields_ = [("arch", C.c_char * 32)] + \
               [(n, C.c_uint32) for n in ("n_layers", "d_model", "d_ff", "n_heads", "n_kv_heads",
                                          "head_dim", "n_ctx", "vocab_size")] + \
               [("rms_eps", C.c_float), ("rope_theta", C.c_float), ("eos", C.c_uint32 * 8),
                ("n_eos", _SZ), ("q_dim", C.c_uint32), ("kv_dim", C.c_uint32)]


def _load_oracle() -> C.CDLL:
    if not os.path.exists(ORACLE_SO):
        raise ImportError(f"{ORACLE_SO} missing: run `make -C oracle`")
    lib = C.CDLL(ORACLE_SO)
    sig = {
        "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
        "orc_dequant_matrix": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P]),
        "orc_matvec": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P]),
        "orc_matmat": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P, _SZ]),
        "orc_matmat_mt": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P, _SZ]),
        "orc_project": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P]),
        "orc_matvec_avx2": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P]),
        "orc_project_avx2": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P]),
        "orc_threads_init": (C.c_int, [C.c_int]),
        "orc_threads_count": (C.c_int, []),
        "orc_threads_shutdown": (None, []),
        "orc_qwen3_new": (_P, [C.POINTER(OrcConfig), C.POINTER(OrcTensor), C.POINTER(OrcTensor),
                               C.POINTER(OrcLayer), C.c_uint32]),
        "orc_qwen3_free": (None, [_P]),
        "orc_qwen3_k_cache": (C.POINTER(C.c_float), [_P]),
        "orc_qwen3_v_cache": (C.POINTER(C.c_float), [_P]),
        "orc_qwen3_set_n_past": (None, [_P, C.c_uint32]),
        "orc_qwen3_n_past": (C.c_uint32, [_P]),
        "orc_qwen3_last_q": (C.POINTER(C.c_float), [_P]),
        "orc_qwen3_last_attn": (C.POINTER(C.c_float), [_P]),
        "orc_qwen3_forward": (C.c_int, [_P, C.c_uint32, _P]),
        "orc_argmax": (C.c_uint32, [_P, _SZ]),
        "orc_sampler_new": (_P, [C.POINTER(SamplerParams), C.c_uint32]),
        "orc_sampler_free": (None, [_P]),
        "orc_sampler_accept": (None, [_P, C.c_uint32]),
        "orc_sampler_sample": (C.c_uint32, [_P, _P]),
        "orc_q8_quantize_block": (C.c_float, [_P, _P, _P]),
        "orc_q4k_int8_dot": (C.c_int32, [_P, _P, C.c_int]),
        "orc_q5k_int8_dot": (C.c_int32, [_P, _P, C.c_int]),
        "orc_q4k_matvec_int8": (C.c_int, [_P, _SZ, _SZ, _P, _P]),
        "orc_q4k_matmat_int8": (C.c_int, [_P, _SZ, _SZ, _P, _P, _SZ]),
        "orc_q5k_matmat_int8": (C.c_int, [_P, _SZ, _SZ, _P, _P, _SZ]),
        "mynah_synth_blocks": (C.c_int, [C.c_int, C.c_uint64, _SZ, _SZ, _SZ, _P, C.c_int]),
        "mynah_synth_normal": (C.c_int, [C.c_uint64, _SZ, C.c_float, C.c_float, _P, C.c_int]),
        "mynah_synth_uniform_u32": (C.c_int, [C.c_uint64, _SZ, C.c_uint32, _P]),
        "mynah_synth_substream": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "mynah_synth_f32_to_f16": (C.c_uint16, [C.c_float]),
        "mynah_synth_qwen3_layout": (C.c_int, [C.POINTER(SynthShape), C.POINTER(SynthTensor), _SZ,
                                               C.POINTER(_SZ), C.POINTER(C.c_uint64)]),
        "mynah_synth_qwen3_fill": (C.c_int, [C.POINTER(SynthShape), C.c_uint64,
                                             C.POINTER(SynthTensor), _SZ, _P, C.c_int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    return lib


orc = _load_oracle()


def load_ref():
    """The compiled reference, or None when it was not built on this machine."""
    if not os.path.exists(REF_SO):
        return None
    lib = C.CDLL(REF_SO)
    sig = {
        "ref_matvec": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P]),
        "ref_matmat": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P, _SZ]),
        "ref_q4_k_matmat_exact": (C.c_int, [_P, _SZ, _SZ, _P, _P, _SZ]),
        "ref_matmat_is_exact": (C.c_int, [_SZ]),
        "ref_dequant_matrix": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P]),
        "ref_dequant": (C.c_int, [C.c_int, _P, _SZ, _P]),
        "ref_write_qwen3_gguf": (C.c_int, [C.c_char_p, C.POINTER(SynthShape),
                                           C.POINTER(SynthTensor), _SZ, _P, C.c_uint32,
                                           C.c_char_p, _SZ]),
        "ref_qwen3_greedy": (C.c_int, [C.c_char_p, _P, _P, C.c_uint32, C.c_uint32, C.c_uint32,
                                       C.c_uint32, C.c_int, _P, _P, C.c_char_p, _SZ]),
        "ref_qwen3_prompt_greedy": (C.c_int, [C.c_char_p, _P, C.c_uint32, C.c_uint32, C.c_uint32,
                                              C.c_int, _P, _P, C.c_char_p, _SZ]),
        "ref_qwen3_run": (C.c_int, [C.c_char_p, _P, _P, C.c_uint32, _P, C.c_uint32, C.c_uint32,
                                    _P, C.c_uint32, C.c_uint32, C.c_int, _P, _P, C.c_char_p,
                                    _SZ]),
        "ref_write_qwen3_gguf_vocab": (C.c_int, [C.c_char_p, C.POINTER(SynthShape),
                                                 C.POINTER(SynthTensor), _SZ, _P, C.c_uint32,
                                                 C.c_char_p, _SZ]),
        "ref_generate_record": (C.c_int, [C.c_char_p, C.c_uint32, _P, _SZ, C.c_uint32, _P, _SZ,
                                          C.c_long, C.c_long, _SZ, _P, _P, _SZ, C.POINTER(_SZ),
                                          _P, _SZ, C.POINTER(_SZ), C.POINTER(C.c_long),
                                          C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                                          C.c_char_p, _SZ]),
        # ingot's GGUF reader (third_party/ingot/include/ingot/gguf.h:60-130)
        "ingot_gguf_open": (C.c_int, [C.POINTER(_P), C.c_char_p, C.c_char_p, _SZ]),
        "ingot_gguf_open_split": (C.c_int, [C.POINTER(_P), C.c_char_p, C.c_char_p, _SZ]),
        "ingot_gguf_close": (None, [_P]),
        "ingot_gguf_version": (C.c_uint32, [_P]),
        "ingot_gguf_alignment": (C.c_uint64, [_P]),
        "ingot_gguf_data_base": (C.c_uint64, [_P, C.c_uint32]),
        "ingot_gguf_count": (_SZ, [_P]),
        "ingot_gguf_at": (C.POINTER(RefTensor), [_P, _SZ]),
        "ingot_gguf_kv_count": (_SZ, [_P]),
        "ingot_gguf_kv_find": (_P, [_P, C.c_char_p]),
        "ingot_kv_u64": (C.c_int, [_P, C.POINTER(C.c_uint64)]),
        "ingot_kv_f64": (C.c_int, [_P, C.POINTER(C.c_double)]),
        "ingot_kv_str": (C.c_int, [_P, C.POINTER(C.c_char_p)]),
        "ingot_kv_arr_len": (C.c_int, [_P, C.POINTER(C.c_uint64)]),
        # the sampler (src/sampler.h:33-43)
        "mynah_slm_sampler_new": (_P, [C.POINTER(SamplerParams), C.c_uint32]),
        "mynah_slm_sampler_free": (None, [_P]),
        "mynah_slm_sampler_accept": (None, [_P, C.c_uint32]),
        "mynah_slm_sample": (C.c_uint32, [_P, _P]),
        # the loader (src/model.h:60-90)
        "mynah_slm_load": (_P, [C.c_char_p, C.c_char_p, _SZ]),
        "mynah_slm_model_config": (C.POINTER(RefConfig), [_P]),
        "mynah_slm_free": (None, [_P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    return lib


def load_ref_int8(sdot: str = "1"):
    """ingot's kernels from an AVX2 + FMA build of the reference sources, with
    the int8 lane switched on for the matvec too (INGOT_SDOT=1, read once by
    the library on its first call; sdot="0" keeps the matvec on its f32 AVX2
    lanes); None when not built on this machine."""
    if not os.path.exists(REF_INT8_SO):
        return None
    os.environ["INGOT_SDOT"] = sdot
    lib = C.CDLL(REF_INT8_SO)
    sig = {
        "ingot_q4_k_matvec": (C.c_int, [_P, _SZ, _SZ, _P, _P]),
        "ingot_q4_k_matvec_int8": (C.c_int, [_P, _SZ, _SZ, _P, _P]),
        "ingot_q4_k_matmat": (C.c_int, [_P, _SZ, _SZ, _P, _P, _SZ]),
        "ingot_q4_k_matmat_exact": (C.c_int, [_P, _SZ, _SZ, _P, _P, _SZ]),
        "ingot_q5_k_matmat": (C.c_int, [_P, _SZ, _SZ, _P, _P, _SZ]),
        "ingot_matmat_is_exact": (C.c_int, [_SZ]),
        "ingot_matvec": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    return lib


def q8_quantize(x: np.ndarray):
    """Oracle quantisation of f32 activations [tokens][cols] (cols % 256 == 0):
    int8 values, per-256 scales [tokens][cols/256], per-32 sums [tokens][cols/32]."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, x.shape[-1])
    tokens, cols = x.shape
    nb = cols // 256
    q = np.empty((tokens, cols), np.int8)
    sc = np.empty((tokens, nb), np.float32)
    sums = np.empty((tokens, nb * 8), np.int32)
    for t in range(tokens):
        for b in range(nb):
            sc[t, b] = orc.orc_q8_quantize_block(x[t, 256 * b:].ctypes.data,
                                                 q[t, 256 * b:].ctypes.data,
                                                 sums[t, 8 * b:].ctypes.data)
    return q, sc, sums


def q4k_int8_dots(w: np.ndarray, rows: int, cols: int, q: np.ndarray) -> np.ndarray:
    """Oracle integer dots: [rows][tokens][cols/32] of the Q4_K quants (0..15)
    with the int8 activations, one per 32-value sub-block."""
    q = np.ascontiguousarray(q, np.int8).reshape(-1, cols)
    nb = cols // 256
    wb = np.ascontiguousarray(w).view(np.uint8).reshape(rows, nb, 144)
    nib = np.empty((rows, nb, 256), np.int32)
    qs = wb[:, :, 16:].astype(np.int32).reshape(rows, nb, 4, 32)
    nib.reshape(rows, nb, 4, 2, 32)[:, :, :, 0] = qs & 15
    nib.reshape(rows, nb, 4, 2, 32)[:, :, :, 1] = qs >> 4
    prod = np.einsum("rbk,tbk->rtbk", nib.reshape(rows, nb, 256),
                     q.astype(np.int32).reshape(-1, nb, 256))
    return prod.reshape(rows, q.shape[0], nb, 8, 32).sum(axis=-1).reshape(rows, q.shape[0], -1)


BLOCK = {12: (256, 144), 13: (256, 176), 14: (256, 210), 8: (32, 34), 2: (32, 18)}


def ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def substream(seed: int, k: int) -> int:
    return int(orc.mynah_synth_substream(seed, k))


def blocks(qtype: int, seed: int, rows: int, cols: int) -> np.ndarray:
    e, b = BLOCK[qtype]
    out = np.empty(rows * (cols // e) * b, np.uint8)
    assert orc.mynah_synth_blocks(qtype, seed, 0, rows, cols, ptr(out), 0) == 0
    return out


def uniform(seed: int, n: int, bound: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    assert orc.mynah_synth_uniform_u32(seed, n, bound, ptr(out)) == 0
    return out


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    assert orc.mynah_synth_normal(seed, n, mean, std, ptr(out), 0) == 0
    return out


def matvec(qtype, w, rows, cols, x) -> np.ndarray:
    y = np.empty(rows, np.float32)
    assert orc.orc_matvec(qtype, ptr(w), rows, cols, ptr(x), ptr(y)) == 0
    return y


def matvec_avx2(qtype, w, rows, cols, x) -> np.ndarray:
    y = np.empty(rows, np.float32)
    assert orc.orc_matvec_avx2(qtype, ptr(w), rows, cols, ptr(x), ptr(y)) == 0
    return y


def project_avx2(qtype, w, rows, cols, x) -> np.ndarray:
    y = np.empty(rows, np.float32)
    assert orc.orc_project_avx2(qtype, ptr(w), rows, cols, ptr(x), ptr(y)) == 0
    return y


def project(qtype, w, rows, cols, x) -> np.ndarray:
    y = np.empty(rows, np.float32)
    assert orc.orc_project(qtype, ptr(w), rows, cols, ptr(x), ptr(y)) == 0
    return y


def matmat(qtype, w, rows, cols, x, tokens, threaded=False) -> np.ndarray:
    y = np.empty(rows * tokens, np.float32)
    fn = orc.orc_matmat_mt if threaded else orc.orc_matmat
    assert fn(qtype, ptr(w), rows, cols, ptr(x), ptr(y), tokens) == 0
    return y


def dequant(qtype, w, rows, cols) -> np.ndarray:
    y = np.empty(rows * cols, np.float32)
    assert orc.orc_dequant_matrix(qtype, ptr(w), rows, cols, ptr(y)) == 0
    return y


# ── random-init Qwen3 (shared layout with the GPU library) ──────────────────

class SynthModel:
    """Host blob + tensor table of a random-init Qwen3 in the Q4_K_M mix."""

    def __init__(self, shape, seed: int = 0):
        self.shape = shape
        self.c_shape = SynthShape(shape.n_layers, shape.d_model, shape.d_ff, shape.n_heads,
                                  shape.n_kv_heads, shape.head_dim, shape.vocab,
                                  shape.rms_eps, shape.rope_theta)
        count, total = _SZ(0), C.c_uint64(0)
        orc.mynah_synth_qwen3_layout(C.byref(self.c_shape), None, 0, C.byref(count),
                                     C.byref(total))
        self.table = (SynthTensor * count.value)()
        assert orc.mynah_synth_qwen3_layout(C.byref(self.c_shape), self.table, count.value,
                                            C.byref(count), C.byref(total)) == 0
        self.count = count.value
        self.blob = np.empty(total.value, np.uint8)
        assert orc.mynah_synth_qwen3_fill(C.byref(self.c_shape), seed, self.table, self.count,
                                          ptr(self.blob), 0) == 0
        self.by_name = {self.table[i].name.decode(): self.table[i] for i in range(self.count)}

    def tensor(self, name: str) -> OrcTensor:
        t = self.by_name[name]
        return OrcTensor(t.type, t.rows, t.cols, ptr(self.blob) + t.offset)


class OracleQwen3:
    """The restated decoder over a SynthModel (same bytes the GPU consumes)."""

    def __init__(self, model: SynthModel, n_ctx: int):
        s = model.shape
        self.model, self.n_ctx = model, n_ctx
        self.cfg = OrcConfig(s.n_layers, s.d_model, s.d_ff, s.n_heads, s.n_kv_heads, s.head_dim,
                             s.vocab, s.rms_eps, s.rope_theta)
        names = ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_q_norm", "attn_k_norm",
                 "attn_output", "ffn_norm", "ffn_gate", "ffn_up", "ffn_down")
        self.layers = (OrcLayer * s.n_layers)()
        for l in range(s.n_layers):
            for field, nm in zip([f[0] for f in OrcLayer._fields_], names):
                setattr(self.layers[l], field, model.tensor(f"blk.{l}.{nm}.weight"))
        self.embed = model.tensor("token_embd.weight")
        self.out_norm = model.tensor("output_norm.weight")
        self.h = orc.orc_qwen3_new(C.byref(self.cfg), C.byref(self.embed), C.byref(self.out_norm),
                                   self.layers, n_ctx)
        assert self.h, "orc_qwen3_new failed"
        self.kv_dim = s.n_kv_heads * s.head_dim

    def prefill_kv(self, k: np.ndarray, v: np.ndarray, n: int) -> None:
        """k, v: [layer][n][kv_dim] f32."""
        s = self.model.shape
        kc = np.ctypeslib.as_array(orc.orc_qwen3_k_cache(self.h),
                                   shape=(s.n_layers, self.n_ctx, self.kv_dim))
        vc = np.ctypeslib.as_array(orc.orc_qwen3_v_cache(self.h),
                                   shape=(s.n_layers, self.n_ctx, self.kv_dim))
        kc[:, :n] = k.reshape(s.n_layers, n, self.kv_dim)
        vc[:, :n] = v.reshape(s.n_layers, n, self.kv_dim)
        orc.orc_qwen3_set_n_past(self.h, n)

    def forward(self, token: int) -> np.ndarray:
        logits = np.empty(self.model.shape.vocab, np.float32)
        assert orc.orc_qwen3_forward(self.h, token, ptr(logits)) == 0
        return logits

    def last_attn(self) -> np.ndarray:
        """The last layer's attention output of the most recent step."""
        s = self.model.shape
        n = s.n_heads * s.head_dim
        return np.ctypeslib.as_array(orc.orc_qwen3_last_attn(self.h), shape=(n,)).copy()

    def last_q(self) -> np.ndarray:
        """The last layer's normalised, rotated query heads of the most recent step."""
        s = self.model.shape
        n = s.n_heads * s.head_dim
        return np.ctypeslib.as_array(orc.orc_qwen3_last_q(self.h), shape=(n,)).copy()

    def greedy(self, first: int, steps: int):
        toks, tok, first_logits = [], first, None
        for i in range(steps):
            lg = self.forward(tok)
            if i == 0:
                first_logits = lg
            tok = int(orc.orc_argmax(ptr(lg), lg.size))
            toks.append(tok)
        return toks, first_logits

    def __del__(self):
        if getattr(self, "h", None):
            orc.orc_qwen3_free(self.h)
            self.h = None


class OracleSampler:
    """The restated sampler (oracle/sampler.c); `sample` and `accept` are C
    function addresses a generation loop can call directly."""

    def __init__(self, vocab: int, **params):
        self.params = sampler_params(**params)
        self.h = orc.orc_sampler_new(C.byref(self.params), vocab)
        assert self.h, "orc_sampler_new failed"

    def sample(self, logits: np.ndarray) -> int:
        """Picks from `logits` (modified in place, as the reference does)."""
        return int(orc.orc_sampler_sample(self.h, ptr(logits)))

    def accept(self, token: int) -> None:
        orc.orc_sampler_accept(self.h, token)

    @staticmethod
    def fn_addresses():
        return (C.cast(orc.orc_sampler_sample, C.c_void_p).value,
                C.cast(orc.orc_sampler_accept, C.c_void_p).value)

    def __del__(self):
        if getattr(self, "h", None):
            orc.orc_sampler_free(self.h)
            self.h = None


def oracle_generate(orc_model: "OracleQwen3", prompt, max_new: int, eos=(), sampler=None,
                    stop_after=None, on_token=None):
    """src/generate.c:13-86 restated over the oracle decoder: the prompt's
    tokens but the last fill the cache, each step forwards the current
    token, picks (greedy, or `sampler`), accepts, stops on an EOS id (which
    counts) or when the token callback asks to (`on_token(id)` true; without
    one, once `stop_after` ids have reached it), and ends early when the
    context is full. Returns the generated ids."""
    for t in prompt[:-1]:
        orc_model.forward(t)
        if sampler:
            sampler.accept(t)
    nxt = prompt[-1]
    if sampler:
        sampler.accept(nxt)
    out, shown = [], 0
    for _ in range(max_new):
        if orc.orc_qwen3_n_past(orc_model.h) >= orc_model.n_ctx:
            break
        lg = orc_model.forward(nxt)
        tok = sampler.sample(lg) if sampler else int(orc.orc_argmax(ptr(lg), lg.size))
        if sampler:
            sampler.accept(tok)
        out.append(tok)
        if tok in eos:
            break
        shown += 1
        if on_token is not None:
            if on_token(tok):
                break
        elif stop_after is not None and shown >= stop_after:
            break
        nxt = tok
    return out


class ChannelRouter:
    """The token callback a front end binds around the generation loop
    (src/generate.c:60-77; oracle/generate_hip.c's token_cb): the think
    markers switch channels and reach neither, answer ids go to `answer`
    (asking to stop once `stop_after` of them arrived, 0: never), ids between
    the markers to `think`. Called with each generated non-EOS id; returns
    whether to stop."""

    def __init__(self, think_open=-1, think_close=-1, stop_after=0):
        self.open, self.close, self.stop_after = think_open, think_close, stop_after
        self.split = think_open >= 0 and think_close >= 0
        self.in_think = False
        self.answer, self.think = [], []

    def __call__(self, tok: int) -> bool:
        if self.split and tok == self.open:
            self.in_think = True
            return False
        if self.split and tok == self.close:
            self.in_think = False
            return False
        if self.in_think:
            self.think.append(tok)
            return False
        self.answer.append(tok)
        return self.stop_after != 0 and len(self.answer) >= self.stop_after


def kv_prefill(substream_fn, shape, config_seed: int, n: int):
    """K and V prefill tensors [layer][n][kv_dim] of a config (see configs.py)."""
    import configs
    return configs.kv_prefill(substream_fn, normal, shape, config_seed, n)


def first_token(config_seed: int, vocab: int) -> int:
    out = np.empty(1, np.uint32)
    assert orc.mynah_synth_uniform_u32(substream(config_seed, 1 << 21), 1, vocab, ptr(out)) == 0
    return int(out[0])


def ref_prompt_greedy(ref, model: SynthModel, prompt, steps, n_ctx, threads=0):
    """The compiled reference's prompt prefill + greedy loop on the same model."""
    p = np.ascontiguousarray(prompt, np.uint32)
    tokens = np.zeros(steps, np.uint32)
    logits = np.zeros(model.shape.vocab, np.float32)
    err = C.create_string_buffer(512)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "model.gguf").encode()
        rc = ref.ref_write_qwen3_gguf(path, C.byref(model.c_shape), model.table, model.count,
                                      ptr(model.blob), n_ctx, err, 512)
        assert rc == 0, err.value
        rc = ref.ref_qwen3_prompt_greedy(path, ptr(p), p.size, steps, n_ctx, threads,
                                         ptr(tokens), ptr(logits), err, 512)
        assert rc == 0, err.value
    return [int(t) for t in tokens], logits


def ref_greedy(ref, model: SynthModel, k, v, n_prefill, first, steps, n_ctx, threads=0):
    """Run the compiled reference loader + decoder on the same model."""
    tokens = np.zeros(steps, np.uint32)
    logits = np.zeros(model.shape.vocab, np.float32)
    err = C.create_string_buffer(512)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "model.gguf").encode()
        rc = ref.ref_write_qwen3_gguf(path, C.byref(model.c_shape), model.table, model.count,
                                      ptr(model.blob), n_ctx, err, 512)
        assert rc == 0, err.value
        rc = ref.ref_qwen3_greedy(path, ptr(k), ptr(v), n_prefill, first, steps, n_ctx, threads,
                                  ptr(tokens), ptr(logits), err, 512)
        assert rc == 0, err.value
    return [int(t) for t in tokens], logits


def ref_run(ref, model: SynthModel, n_ctx, steps, k=None, v=None, n_prefill=0, prompt=None,
            first=0, inputs=None, want_logits=True, threads=0):
    """The compiled reference decoder (ref_harness.c ref_qwen3_run): greedy
    ids of every step and, optionally, every step's logits [steps][vocab]."""
    greedy = np.zeros(steps, np.uint32)
    logits = np.zeros((steps, model.shape.vocab), np.float32) if want_logits else None
    p = np.ascontiguousarray(prompt if prompt is not None else [], np.uint32)
    f = np.ascontiguousarray(inputs, np.uint32) if inputs is not None else None
    err = C.create_string_buffer(512)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "model.gguf").encode()
        rc = ref.ref_write_qwen3_gguf(path, C.byref(model.c_shape), model.table, model.count,
                                      ptr(model.blob), n_ctx, err, 512)
        assert rc == 0, err.value
        rc = ref.ref_qwen3_run(path, ptr(k) if n_prefill else None,
                               ptr(v) if n_prefill else None, n_prefill,
                               ptr(p) if p.size else None, p.size, first,
                               ptr(f) if f is not None else None, steps, n_ctx, threads,
                               ptr(greedy), ptr(logits) if want_logits else None, err, 512)
        assert rc == 0, err.value
    return [int(t) for t in greedy], logits


def ref_generate(ref, model: SynthModel, n_ctx, prompt, max_new, eos=(), think=(-1, -1),
                 stop_after=0, sampler=None):
    """src/generate.c:13-86 compiled (ref_harness.c ref_generate_record) on
    the model written with a vocabulary: the ids its answer and thinking
    callbacks saw, the count it returned, the timing's generated count and
    the state's position afterwards. `sampler`: None for greedy, else the
    sampler_params keyword arguments."""
    p = np.ascontiguousarray(prompt, np.uint32)
    e = np.ascontiguousarray(list(eos) or [0], np.uint32)
    ans = np.zeros(max_new + 1, np.uint32)
    thk = np.zeros(max_new + 1, np.uint32)
    n_ans, n_thk = _SZ(0), _SZ(0)
    produced, n_gen, n_past = C.c_long(0), C.c_uint32(0), C.c_uint32(0)
    sp = sampler_params(**sampler) if sampler is not None else None
    err = C.create_string_buffer(512)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "model.gguf").encode()
        rc = ref.ref_write_qwen3_gguf_vocab(path, C.byref(model.c_shape), model.table,
                                            model.count, ptr(model.blob), n_ctx, err, 512)
        assert rc == 0, err.value
        rc = ref.ref_generate_record(path, n_ctx, ptr(p), p.size, max_new, ptr(e), len(eos),
                                     think[0], think[1], stop_after,
                                     C.cast(C.byref(sp), C.c_void_p) if sp is not None else None,
                                     ptr(ans), ans.size, C.byref(n_ans), ptr(thk), thk.size,
                                     C.byref(n_thk), C.byref(produced), C.byref(n_gen),
                                     C.byref(n_past), err, 512)
        assert rc == 0, err.value
    return {"answer": [int(t) for t in ans[:n_ans.value]],
            "think": [int(t) for t in thk[:n_thk.value]],
            "produced": int(produced.value), "n_gen": int(n_gen.value),
            "n_past": int(n_past.value)}


def ref_gguf_read(ref, path: str, keys=(), split: bool = False):
    """What the reference's reader makes of the file at `path`: None when
    ingot_gguf_open (split: ingot_gguf_open_split) refuses it, else its
    header, tensor table (split: each row also carrying the tensor's shard)
    and, for each of `keys`, the u64 / f64 / string / array-length reads
    (None where refused)."""
    g = _P()
    err = C.create_string_buffer(512)
    opener = ref.ingot_gguf_open_split if split else ref.ingot_gguf_open
    if opener(C.byref(g), os.fsencode(path), err, 512) != 0:
        assert g.value is None and err.value
        return None
    try:
        out = {"version": int(ref.ingot_gguf_version(g)), "n_kv": int(ref.ingot_gguf_kv_count(g)),
               "alignment": int(ref.ingot_gguf_alignment(g)),
               "data_base": int(ref.ingot_gguf_data_base(g, 0)), "tensors": [], "kv": {}}
        for i in range(ref.ingot_gguf_count(g)):
            t = ref.ingot_gguf_at(g, i).contents
            row = [t.name.decode(), t.type, t.rank, list(t.ne[:t.rank]), int(t.offset),
                   int(t.nbytes)]
            out["tensors"].append(row + [int(t.shard)] if split else row)
        for key in keys:
            kv = ref.ingot_gguf_kv_find(g, key.encode())
            if not kv:
                out["kv"][key] = None
                continue
            u, f, sp, n = C.c_uint64(), C.c_double(), C.c_char_p(), C.c_uint64()
            out["kv"][key] = {
                "u64": int(u.value) if ref.ingot_kv_u64(kv, C.byref(u)) == 0 else None,
                "f64": float(f.value) if ref.ingot_kv_f64(kv, C.byref(f)) == 0 else None,
                "str": sp.value.decode() if ref.ingot_kv_str(kv, C.byref(sp)) == 0 else None,
                "arr_len": int(n.value) if ref.ingot_kv_arr_len(kv, C.byref(n)) == 0 else None}
        return out
    finally:
        ref.ingot_gguf_close(g)


def ref_qwen3_config(ref, path: str):
    """mynah_slm_load's config for the file, or None when it refuses it."""
    err = C.create_string_buffer(512)
    m = ref.mynah_slm_load(os.fsencode(path), err, 512)
    if not m:
        assert err.value
        return None
    try:
        c = ref.mynah_slm_model_config(m).contents
        return {"n_layers": c.n_layers, "d_model": c.d_model, "d_ff": c.d_ff,
                "n_heads": c.n_heads, "n_kv_heads": c.n_kv_heads, "head_dim": c.head_dim,
                "n_ctx": c.n_ctx, "vocab": c.vocab_size, "rms_eps": float(c.rms_eps),
                "rope_theta": float(c.rope_theta)}
    finally:
        ref.mynah_slm_free(m)
