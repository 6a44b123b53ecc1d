"""ctypes binding of libmynah_hip.so (the gfx950 kernels behind include/kernels_hip.h).

The library is C11 + HIP; this module only loads it and gives numpy-friendly
wrappers to tests and the benchmark. It never falls back to anything: if the
shared library is missing, importing it raises.
"""
from __future__ import annotations

import ctypes as C
import os
import types

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# MYNAH_HIP_LIB names another build of the library (e.g. a tuning variant).
LIB_PATH = os.environ.get("MYNAH_HIP_LIB") or os.path.join(HERE, "libmynah_hip.so")

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 8, 12, 13, 14
BLOCK = {Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_0: (32, 34), Q4_0: (32, 18)}

_P = C.c_void_p
_SZ = C.c_size_t


class Qwen3Shape(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("n_layers", "d_model", "d_ff", "n_heads", "n_kv_heads",
                                          "head_dim", "vocab")] + \
               [("rms_eps", C.c_float), ("rope_theta", C.c_float)]


class SynthTensor(C.Structure):
    _fields_ = [("name", C.c_char * 48), ("type", C.c_int), ("rank", C.c_uint32),
                ("rows", C.c_uint64), ("cols", C.c_uint64), ("offset", C.c_uint64),
                ("nbytes", C.c_uint64)]


class GenParams(C.Structure):
    """mynah_hip_gen_params (include/mynah_generate.h); the callbacks are
    plain function addresses."""
    _fields_ = [("prompt", C.c_void_p), ("n_prompt", C.c_size_t), ("max_new", C.c_uint32),
                ("eos", C.c_void_p), ("n_eos", C.c_size_t), ("on_token", C.c_void_p),
                ("token_ctx", C.c_void_p), ("sample", C.c_void_p), ("accept", C.c_void_p),
                ("sampler", C.c_void_p), ("chunk", C.c_uint32), ("device_sampler", C.c_void_p)]


class SamplerParams(C.Structure):
    """mynah_hip_sampler_params (include/mynah_generate.h) = the reference's
    mynah_slm_sampler_params (src/sampler.h:16-30)."""
    _fields_ = [("temp", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float),
                ("min_p", C.c_float), ("repeat_penalty", C.c_float), ("freq_penalty", C.c_float),
                ("presence_penalty", C.c_float), ("penalty_window", C.c_uint32),
                ("seed", C.c_uint64)]


class GenTiming(C.Structure):
    """mynah_hip_timing (include/mynah_generate.h)."""
    _fields_ = [("prefill_s", C.c_double), ("decode_s", C.c_double), ("ttft_s", C.c_double),
                ("n_prompt", C.c_uint32), ("n_gen", C.c_uint32), ("ttft_done", C.c_int)]


TOKEN_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32)


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built: run `make -C mynah-slm_amd` (or __graft_entry__.build())")
    lib = C.CDLL(LIB_PATH)
    sig = {
        "ingot_matvec": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P]),
        "ingot_matmat": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P, _SZ]),
        "ingot_dequant_matrix": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P]),
        "ingot_has_kernel": (C.c_int, [C.c_int]),
        "ingot_matmat_is_exact": (C.c_int, [_SZ]),
        "ingot_q4_k_matmat_exact": (C.c_int, [_P, _SZ, _SZ, _P, _P, _SZ]),
        "ingot_q4_k_matvec_int8": (C.c_int, [_P, _SZ, _SZ, _P, _P]),
        "ingot_q4_k_matvec_scalar": (C.c_int, [_P, _SZ, _SZ, _P, _P]),
        "ingot_gguf_matvec": (C.c_int, [_P, _P, _P, _P]),
        "ingot_gguf_matmat": (C.c_int, [_P, _P, _P, _P, _SZ]),
        "ingot_gguf_dequant_matrix": (C.c_int, [_P, _P, _P]),
        "ingot_q5_k_matvec_scalar": (C.c_int, [_P, _SZ, _SZ, _P, _P]),
        "ingot_q5_k_matmat_exact": (C.c_int, [_P, _SZ, _SZ, _P, _P, _SZ]),
        "mynah_hip_set_int8": (C.c_int, [C.c_int]),
        "mynah_hip_int8": (C.c_int, []),
        "mynah_hip_q8_quantize_dev": (C.c_int, [_P, _SZ, _SZ, _P, _P, _P, _P]),
        "mynah_hip_q4k_int8_dev": (C.c_int, [_P, _SZ, _SZ, _P, _P, _P, _P, _SZ, _P]),
        "mynah_hip_int8_product_noalloc_dev": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P, _SZ,
                                                         _P]),
        "mynah_hip_init": (C.c_int, [C.c_int]),
        "mynah_hip_last_error": (C.c_char_p, []),
        "mynah_hip_register": (C.c_int, [_P, _SZ]),
        "mynah_hip_unregister": (C.c_int, [_P]),
        "mynah_hip_device_ptr": (_P, [_P]),
        "mynah_hip_matvec_dev": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P, _P]),
        "mynah_hip_matmat_dev": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P, _SZ, _P]),
        "mynah_hip_dequant_dev": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P]),
        "mynah_hip_matmat_mv_dev": (C.c_int, [C.c_int, _P, _SZ, _SZ, _P, _P, _SZ, _P, _P]),
        "mynah_hip_alloc": (_P, [_SZ]),
        "mynah_hip_free": (C.c_int, [_P]),
        "mynah_hip_h2d": (C.c_int, [_P, _P, _SZ]),
        "mynah_hip_d2h": (C.c_int, [_P, _P, _SZ]),
        "mynah_hip_memset": (C.c_int, [_P, C.c_int, _SZ]),
        "mynah_hip_sync": (C.c_int, [_P]),
        "mynah_hip_stream": (_P, []),
        "mynah_hip_set_gemv_order": (C.c_int, [C.c_int]),
        "mynah_hip_set_index_order_sums": (C.c_int, [C.c_int]),
        "mynah_hip_gemv_order": (C.c_int, []),
        "mynah_hip_gemv_kernel": (C.c_char_p, [C.c_int, C.c_size_t, C.c_size_t, C.c_int]),
        "mynah_hip_event_create": (_P, []),
        "mynah_hip_event_record": (C.c_int, [_P, _P]),
        "mynah_hip_event_elapsed": (C.c_int, [_P, _P, C.POINTER(C.c_float)]),
        "mynah_hip_event_destroy": (C.c_int, [_P]),
        "mynah_hip_copy_dev": (C.c_int, [_P, _P, _SZ, _P]),
        "mynah_hip_read_dev": (C.c_int, [_P, _SZ, _P, _P]),
        "mynah_hip_mfma_probe": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, C.c_uint32, _P]),
        "mynah_hip_valu_add_rate": (C.c_int, [C.c_uint32, C.POINTER(C.c_float),
                                              C.POINTER(C.c_uint32)]),
        "mynah_hip_expf_dev": (C.c_int, [_P, _P, _SZ, _P]),
        "mynah_hip_time_sweep": (C.c_int, [C.c_int, _P, _P, C.c_int, _P, _P, _P, _P, C.c_int,
                                           C.c_int, C.c_int, C.POINTER(C.c_float),
                                           C.POINTER(C.c_float)]),
        "mynah_hip_time_matvec": (C.c_int, [C.c_int, _P, C.c_int, _SZ, _SZ, _P, _P, C.c_int,
                                            C.POINTER(C.c_float)]),
        "mynah_synth_blocks": (C.c_int, [C.c_int, C.c_uint64, _SZ, _SZ, _SZ, _P, C.c_int]),
        "mynah_synth_normal": (C.c_int, [C.c_uint64, _SZ, C.c_float, C.c_float, _P, C.c_int]),
        "mynah_synth_uniform_u32": (C.c_int, [C.c_uint64, _SZ, C.c_uint32, _P]),
        "mynah_synth_substream": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "mynah_synth_f32_to_f16": (C.c_uint16, [C.c_float]),
        "mynah_synth_qwen3_layout": (C.c_int, [C.POINTER(Qwen3Shape), C.POINTER(SynthTensor), _SZ,
                                               C.POINTER(_SZ), C.POINTER(C.c_uint64)]),
        "mynah_synth_qwen3_fill": (C.c_int, [C.POINTER(Qwen3Shape), C.c_uint64,
                                             C.POINTER(SynthTensor), _SZ, _P, C.c_int]),
        "mynah_hip_qwen3_new": (_P, [C.POINTER(Qwen3Shape), C.POINTER(SynthTensor), _SZ, _P,
                                     C.c_uint64, C.c_uint32, C.c_char_p, _SZ]),
        "mynah_hip_qwen3_free": (None, [_P]),
        "mynah_hip_qwen3_reset": (None, [_P]),
        "mynah_hip_qwen3_forward": (C.c_int, [_P, C.c_uint32, _P]),
        "mynah_hip_qwen3_generate": (C.c_int, [_P, C.c_uint32, C.c_uint32, _P,
                                               C.POINTER(C.c_float)]),
        "mynah_hip_qwen3_forced": (C.c_int, [_P, _P, C.c_uint32, _P, _P]),
        "mynah_hip_sampler_new": (_P, [C.POINTER(SamplerParams), C.c_uint32]),
        "mynah_hip_sampler_free": (None, [_P]),
        "mynah_hip_sampler_accept": (C.c_int, [_P, C.c_uint32]),
        "mynah_hip_sample": (C.c_int, [_P, _P, C.POINTER(C.c_uint32)]),
        "mynah_hip_qwen3_generate_tokens": (C.c_long, [_P, C.POINTER(GenParams),
                                                       C.POINTER(GenTiming)]),
        "mynah_hip_qwen3_set_kv": (C.c_int, [_P, _P, _P, C.c_uint32]),
        "mynah_hip_qwen3_get_kv": (C.c_int, [_P, _P, _P, C.c_uint32]),
        "mynah_hip_qwen3_prefill": (C.c_int, [_P, _P, C.c_uint32]),
        "mynah_hip_qwen3_set_prefill": (C.c_int, [_P, C.c_int]),
        "mynah_hip_qwen3_n_past": (C.c_uint32, [_P]),
        "mynah_hip_qwen3_read_attn": (C.c_int, [_P, _P]),
        "mynah_hip_qwen3_uses_graph": (C.c_int, [_P]),
        "mynah_hip_qwen3_set_attention": (C.c_int, [_P, C.c_int]),
        "mynah_hip_qwen3_prompt": (C.c_int, [_P, _P, C.c_uint32, C.c_uint32, _P,
                                             C.POINTER(C.c_float), C.POINTER(C.c_float)]),
        "mynah_gguf_open": (_P, [C.c_char_p, C.c_char_p, _SZ]),
        "mynah_gguf_open_split": (_P, [C.c_char_p, C.c_char_p, _SZ]),
        "mynah_gguf_n_shards": (C.c_uint32, [_P]),
        "mynah_gguf_shard_data": (_P, [_P, C.c_uint32, C.POINTER(C.c_uint64),
                                       C.POINTER(C.c_uint64)]),
        "mynah_gguf_tensor_place": (C.c_int, [_P, C.c_uint64, C.POINTER(C.c_uint32),
                                              C.POINTER(C.c_uint64)]),
        "mynah_gguf_close": (None, [_P]),
        "mynah_gguf_version": (C.c_uint32, [_P]),
        "mynah_gguf_alignment": (C.c_uint64, [_P]),
        "mynah_gguf_n_kv": (C.c_uint64, [_P]),
        "mynah_gguf_n_tensors": (C.c_uint64, [_P]),
        "mynah_gguf_kv_u64": (C.c_int, [_P, C.c_char_p, C.POINTER(C.c_uint64)]),
        "mynah_gguf_kv_f64": (C.c_int, [_P, C.c_char_p, C.POINTER(C.c_double)]),
        "mynah_gguf_kv_str": (C.c_int, [_P, C.c_char_p, C.POINTER(C.c_void_p), C.POINTER(_SZ)]),
        "mynah_gguf_kv_arr_len": (C.c_int, [_P, C.c_char_p, C.POINTER(C.c_uint64)]),
        "mynah_gguf_qwen3_shape": (C.c_int, [_P, C.POINTER(Qwen3Shape), C.POINTER(C.c_uint32),
                                             C.c_char_p, _SZ]),
        "mynah_gguf_tensor_table": (C.c_int, [_P, C.POINTER(SynthTensor), _SZ, C.POINTER(_SZ)]),
        "mynah_gguf_data": (_P, [_P, C.POINTER(C.c_uint64)]),
        "mynah_hip_qwen3_from_gguf": (_P, [C.c_char_p, C.c_uint32, C.c_char_p, _SZ]),
    }
    # The per-type kernels of quant.h: matvec(w, rows, cols, x, y),
    # dequant(w, rows, cols, y), matmat(w, rows, cols, x, y, tokens).
    for prefix in ("q4_k", "q5_k", "q6_k", "q8_0", "q4_0"):
        sig[f"ingot_{prefix}_matvec"] = (C.c_int, [_P, _SZ, _SZ, _P, _P])
        sig[f"ingot_{prefix}_dequant"] = (C.c_int, [_P, _SZ, _SZ, _P])
        if prefix != "q4_0":
            sig[f"ingot_{prefix}_matmat"] = (C.c_int, [_P, _SZ, _SZ, _P, _P, _SZ])
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib, frozenset(sig)


# SIGNATURES: every entry point given restype / argtypes above. ctypes passes
# an undeclared pointer argument as a C int (the upper 32 bits lost), so
# nothing may call the library through a name outside this set.
lib, SIGNATURES = _load()


class HipError(RuntimeError):
    pass


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        raise HipError(f"{what}: {lib.mynah_hip_last_error().decode(errors='replace')}")


def ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def row_bytes(qtype: int, cols: int) -> int:
    elems, nbytes = BLOCK[qtype]
    return cols // elems * nbytes


# ── synthetic inputs (shared generator, see include/mynah_synth.h) ──────────

def synth_blocks(qtype: int, seed: int, rows: int, cols: int, row0: int = 0) -> np.ndarray:
    out = np.empty(rows * row_bytes(qtype, cols), dtype=np.uint8)
    if lib.mynah_synth_blocks(qtype, seed, row0, rows, cols, ptr(out), 0) != 0:
        raise ValueError("synth_blocks: bad arguments")
    return out


def synth_normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    if lib.mynah_synth_normal(seed, n, mean, std, ptr(out), 0) != 0:
        raise ValueError("synth_normal: bad arguments")
    return out


def substream(seed: int, k: int) -> int:
    return int(lib.mynah_synth_substream(seed, k))


# ── device memory ───────────────────────────────────────────────────────────

class DeviceBuffer:
    """A plain hipMalloc allocation owned by the library."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = lib.mynah_hip_alloc(self.nbytes)
        if not p:
            raise HipError(f"alloc({nbytes}): {lib.mynah_hip_last_error().decode()}")
        self.ptr = int(p)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        check(lib.mynah_hip_h2d(b.ptr, ptr(a), a.nbytes), "h2d")
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(lib.mynah_hip_h2d(self.ptr + offset, ptr(a), a.nbytes), "h2d")

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(lib.mynah_hip_d2h(ptr(out), self.ptr + offset, out.nbytes), "d2h")
        return out

    def free(self) -> None:
        if self.ptr:
            check(lib.mynah_hip_free(self.ptr), "free")
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sync() -> None:
    check(lib.mynah_hip_sync(None), "sync")


# ── kernels through the drop-in (host pointer) ABI ──────────────────────────

def matvec(qtype: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    y = np.empty(rows, dtype=np.float32)
    check(lib.ingot_matvec(qtype, ptr(w), rows, cols, ptr(x), ptr(y)), "ingot_matvec")
    return y


def matmat(qtype: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray, tokens: int) -> np.ndarray:
    y = np.empty(tokens * rows, dtype=np.float32)
    check(lib.ingot_matmat(qtype, ptr(w), rows, cols, ptr(x), ptr(y), tokens), "ingot_matmat")
    return y


INT8_OFF, INT8_BATCHED, INT8_ALL = 0, 1, 2


def set_int8(mode: int) -> None:
    """The int8 activation lane (INT8_OFF, INT8_BATCHED, INT8_ALL): batched
    Q4_K and Q5_K products, and with INT8_ALL also the Q4_K matvec."""
    check(lib.mynah_hip_set_int8(mode), "set_int8")


def matvec_int8(w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    y = np.empty(rows, dtype=np.float32)
    check(lib.ingot_q4_k_matvec_int8(ptr(w), rows, cols, ptr(x), ptr(y)), "q4_k_matvec_int8")
    return y


def matmat_exact(w: np.ndarray, rows: int, cols: int, x: np.ndarray, tokens: int) -> np.ndarray:
    y = np.empty(tokens * rows, dtype=np.float32)
    check(lib.ingot_q4_k_matmat_exact(ptr(w), rows, cols, ptr(x), ptr(y), tokens),
          "q4_k_matmat_exact")
    return y


def q8_quantize_dev(x: int, tokens: int, cols: int, xq: int, xs: int, xsum: int,
                    stream=None) -> None:
    check(lib.mynah_hip_q8_quantize_dev(x, tokens, cols, xq, xs, xsum, stream), "q8_quantize")


def q4k_int8_dev(w: int, rows: int, cols: int, xq: int, xs: int, xsum: int, y: int,
                 tokens: int, stream=None) -> None:
    check(lib.mynah_hip_q4k_int8_dev(w, rows, cols, xq, xs, xsum, y, tokens, stream),
          "q4k_int8")


def matmat_mv(qtype: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray, tokens: int,
              res: np.ndarray = None) -> np.ndarray:
    """Y[tokens][rows] in the matvec summation order (+ res), via the GPU."""
    wd, xd = DeviceBuffer.from_array(w), DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    yd = DeviceBuffer.from_array(np.ascontiguousarray(res, np.float32)) if res is not None \
        else DeviceBuffer(4 * rows * tokens)
    try:
        check(lib.mynah_hip_matmat_mv_dev(qtype, wd.ptr, rows, cols, xd.ptr, yd.ptr, tokens,
                                          yd.ptr if res is not None else None, None), "matmat_mv")
        sync()
        return yd.download(np.float32, rows * tokens)
    finally:
        for b in (wd, xd, yd):
            b.free()


def dequant(qtype: int, w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    y = np.empty(rows * cols, dtype=np.float32)
    check(lib.ingot_dequant_matrix(qtype, ptr(w), rows, cols, ptr(y)), "ingot_dequant_matrix")
    return y


# ── device-pointer twins ────────────────────────────────────────────────────

def matvec_dev(qtype: int, w: int, rows: int, cols: int, x: int, y: int, stream=None) -> None:
    check(lib.mynah_hip_matvec_dev(qtype, w, rows, cols, x, y, stream), "matvec_dev")


def matmat_dev(qtype: int, w: int, rows: int, cols: int, x: int, y: int, tokens: int,
               stream=None) -> None:
    check(lib.mynah_hip_matmat_dev(qtype, w, rows, cols, x, y, tokens, stream), "matmat_dev")


def dequant_dev(qtype: int, w: int, rows: int, cols: int, y: int, stream=None) -> None:
    check(lib.mynah_hip_dequant_dev(qtype, w, rows, cols, y, stream), "dequant_dev")


def copy_dev(dst: int, src: int, nbytes: int, stream=None) -> None:
    check(lib.mynah_hip_copy_dev(dst, src, nbytes, stream), "copy_dev")


def read_dev(src: int, nbytes: int, sink: int, stream=None) -> None:
    check(lib.mynah_hip_read_dev(src, nbytes, sink, stream), "read_dev")


def valu_add_rate(iters: int = 20000):
    """(ns per wave64 v_add_f32 per SIMD with every SIMD issuing only f32
    adds, the device's SIMD count)."""
    ns, simds = C.c_float(0.0), C.c_uint32(0)
    check(lib.mynah_hip_valu_add_rate(iters, C.byref(ns), C.byref(simds)), "valu_add_rate")
    return float(ns.value), int(simds.value)


def time_sweep(mats, w_ptrs, copies: int, x_ptrs, y_ptrs, steps: int, timed: int,
               every: int = 1):
    """Time `steps` passes over mats (launched from C); returns (total ms,
    average ms of matrix `timed`'s launch over every `every`-th pass). w_ptrs
    is [matrix][copy] flattened."""
    n = len(mats)
    types = (C.c_int * n)(*[m.qtype for m in mats])
    rows = (C.c_size_t * n)(*[m.rows for m in mats])
    cols = (C.c_size_t * n)(*[m.cols for m in mats])
    w = (C.c_void_p * len(w_ptrs))(*w_ptrs)
    x = (C.c_void_p * n)(*x_ptrs)
    y = (C.c_void_p * n)(*y_ptrs)
    tot, tim = C.c_float(0.0), C.c_float(0.0)
    check(lib.mynah_hip_time_sweep(n, types, w, copies, rows, cols, x, y, steps, timed, every,
                                   C.byref(tot), C.byref(tim)), "time_sweep")
    return float(tot.value), float(tim.value)


def gemv_kernel(qtype: int, rows: int, cols: int, order: int = -1) -> str:
    """Name of the kernel one matvec of this shape launches (the plan only)."""
    name = lib.mynah_hip_gemv_kernel(qtype, rows, cols, order)
    if name is None:
        raise HipError(f"gemv_kernel: {lib.mynah_hip_last_error().decode(errors='replace')}")
    return name.decode()


def time_matvec(qtype: int, w_ptrs, rows: int, cols: int, x: int, y: int, iters: int) -> float:
    arr = (C.c_void_p * len(w_ptrs))(*w_ptrs)
    ms = C.c_float(0.0)
    check(lib.mynah_hip_time_matvec(qtype, C.cast(arr, C.c_void_p), len(w_ptrs), rows, cols,
                                    x, y, iters, C.byref(ms)), "time_matvec")
    return float(ms.value)


class Event:
    """A HIP event on the library's stream (or a given one)."""

    def __init__(self):
        p = lib.mynah_hip_event_create()
        if not p:
            raise HipError(lib.mynah_hip_last_error().decode())
        self.p = p

    def record(self, stream=None) -> None:
        check(lib.mynah_hip_event_record(self.p, stream), "event_record")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0.0)
        check(lib.mynah_hip_event_elapsed(self.p, end.p, C.byref(ms)), "event_elapsed")
        return float(ms.value)

    def __del__(self):
        try:
            lib.mynah_hip_event_destroy(self.p)
        except Exception:
            pass


# ── random-init Qwen3 and the resident decoder ──────────────────────────────

class SynthQwen3:
    """Tensor table + host blob of a random-init Qwen3 (include/mynah_synth.h)."""

    def __init__(self, shape, seed: int = 0):
        self.shape = shape
        self.c_shape = Qwen3Shape(shape.n_layers, shape.d_model, shape.d_ff, shape.n_heads,
                                  shape.n_kv_heads, shape.head_dim, shape.vocab, shape.rms_eps,
                                  shape.rope_theta)
        count, total = _SZ(0), C.c_uint64(0)
        lib.mynah_synth_qwen3_layout(C.byref(self.c_shape), None, 0, C.byref(count), C.byref(total))
        self.table = (SynthTensor * count.value)()
        if lib.mynah_synth_qwen3_layout(C.byref(self.c_shape), self.table, count.value,
                                        C.byref(count), C.byref(total)) != 0:
            raise ValueError("bad Qwen3 shape")
        self.count = count.value
        self.blob = np.empty(total.value, np.uint8)
        if lib.mynah_synth_qwen3_fill(C.byref(self.c_shape), seed, self.table, self.count,
                                      ptr(self.blob), 0) != 0:
            raise ValueError("synthesis failed")

    def weight_bytes(self) -> int:
        return int(sum(self.table[i].nbytes for i in range(self.count)))


class GgufShape:
    """A Qwen3 config read from a GGUF file (the fields of Qwen3Shape)."""

    def __init__(self, c: Qwen3Shape):
        for name, _ in Qwen3Shape._fields_:
            setattr(self, name, getattr(c, name))


class GgufFile:
    """A memory-mapped GGUF v2 / v3 file (include/mynah_gguf.h)."""

    def __init__(self, path: str, split: bool = False):
        """split: open a <prefix>-0000k-of-0000n.gguf checkpoint whole
        (mynah_gguf_open_split)."""
        err = C.create_string_buffer(512)
        fn = lib.mynah_gguf_open_split if split else lib.mynah_gguf_open
        self.h = fn(os.fsencode(path), err, 512)
        if not self.h:
            raise HipError(f"gguf_open: {err.value.decode(errors='replace')}")

    @property
    def n_shards(self) -> int:
        return int(lib.mynah_gguf_n_shards(self.h))

    def places(self):
        """[(shard, offset within the shard's data section)] of every tensor."""
        out, sh, off = [], C.c_uint32(), C.c_uint64()
        for i in range(self.n_tensors):
            check(lib.mynah_gguf_tensor_place(self.h, i, C.byref(sh), C.byref(off)), "place")
            out.append((int(sh.value), int(off.value)))
        return out

    def shard_size(self, shard: int) -> int:
        """Bytes of shard `shard`'s data section (to the end of its file)."""
        size, at = C.c_uint64(), C.c_uint64()
        if not lib.mynah_gguf_shard_data(self.h, shard, C.byref(size), C.byref(at)):
            raise HipError("shard_size: no such shard")
        return int(size.value)

    def shard_bytes(self, shard: int, offset: int, nbytes: int) -> bytes:
        """nbytes of shard `shard`'s data section from `offset`."""
        size, at = C.c_uint64(), C.c_uint64()
        p = lib.mynah_gguf_shard_data(self.h, shard, C.byref(size), C.byref(at))
        if not p or offset + nbytes > size.value:
            raise HipError("shard_bytes: out of range")
        return C.string_at(p + offset, nbytes)

    @property
    def version(self) -> int:
        return int(lib.mynah_gguf_version(self.h))

    @property
    def alignment(self) -> int:
        return int(lib.mynah_gguf_alignment(self.h))

    @property
    def n_kv(self) -> int:
        return int(lib.mynah_gguf_n_kv(self.h))

    @property
    def n_tensors(self) -> int:
        return int(lib.mynah_gguf_n_tensors(self.h))

    def get_int(self, key: str):
        v = C.c_uint64(0)
        return int(v.value) if lib.mynah_gguf_kv_u64(self.h, key.encode(), C.byref(v)) == 0 else None

    def get_float(self, key: str):
        v = C.c_double(0.0)
        return float(v.value) if lib.mynah_gguf_kv_f64(self.h, key.encode(), C.byref(v)) == 0 else None

    def get_str(self, key: str):
        p, n = C.c_void_p(), _SZ(0)
        if lib.mynah_gguf_kv_str(self.h, key.encode(), C.byref(p), C.byref(n)) != 0:
            return None
        return C.string_at(p.value, n.value).decode("utf-8", errors="replace") if n.value else ""

    def array_len(self, key: str):
        v = C.c_uint64(0)
        return int(v.value) if lib.mynah_gguf_kv_arr_len(self.h, key.encode(), C.byref(v)) == 0 else None

    def qwen3_shape(self):
        """(GgufShape, context_length) the way the reference's loader reads them."""
        c, n_ctx, err = Qwen3Shape(), C.c_uint32(0), C.create_string_buffer(512)
        if lib.mynah_gguf_qwen3_shape(self.h, C.byref(c), C.byref(n_ctx), err, 512) != 0:
            raise HipError(f"gguf config: {err.value.decode(errors='replace')}")
        return GgufShape(c), int(n_ctx.value)

    def tensors(self):
        """[(name, ggml type, rank, rows, cols, offset, nbytes)] in file order."""
        n = _SZ(0)
        check(lib.mynah_gguf_tensor_table(self.h, None, 0, C.byref(n)), "gguf tensors")
        table = (SynthTensor * max(n.value, 1))()
        check(lib.mynah_gguf_tensor_table(self.h, table, n.value, C.byref(n)), "gguf tensors")
        return [(t.name.decode(errors="replace"), t.type, t.rank, t.rows, t.cols, t.offset,
                 t.nbytes)
                for t in table[:n.value]]

    def data_bytes(self) -> int:
        """Bytes from the start of the data section to the end of the file."""
        n = C.c_uint64(0)
        lib.mynah_gguf_data(self.h, C.byref(n))
        return int(n.value)

    def tensor_data(self, offset: int, nbytes: int) -> bytes:
        """A copy of `nbytes` of the data section from `offset`."""
        n = C.c_uint64(0)
        base = lib.mynah_gguf_data(self.h, C.byref(n))
        if offset < 0 or nbytes < 0 or offset + nbytes > n.value:
            raise ValueError("range outside the data section")
        return C.string_at(base + offset, nbytes)

    def close(self) -> None:
        if self.h:
            lib.mynah_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


ATTN_EXACT, ATTN_SPLIT = 0, 1
PREFILL_BATCHED, PREFILL_STEPS = 0, 1


def sampler_params(temp=0.0, top_k=0, top_p=1.0, min_p=0.0, repeat_penalty=1.0,
                   freq_penalty=0.0, presence_penalty=0.0, penalty_window=64, seed=0):
    return SamplerParams(temp, top_k, top_p, min_p, repeat_penalty, freq_penalty,
                         presence_penalty, penalty_window, seed)


class DeviceSampler:
    """The reference's sampler on the device (mynah_hip_sampler_*): `sample`
    picks from host logits (modified in place like the reference's), and
    Qwen3Decoder.generate_tokens(device_sampler=...) samples inside the
    captured steps."""

    def __init__(self, vocab: int, **params):
        self.params = sampler_params(**params)
        self.h = lib.mynah_hip_sampler_new(C.byref(self.params), vocab)
        if not self.h:
            raise HipError(f"sampler_new: {lib.mynah_hip_last_error().decode()}")

    def sample(self, logits: np.ndarray) -> int:
        out = C.c_uint32(0)
        check(lib.mynah_hip_sample(self.h, ptr(logits), C.byref(out)), "sample")
        return int(out.value)

    def accept(self, token: int) -> None:
        check(lib.mynah_hip_sampler_accept(self.h, token), "sampler_accept")

    def close(self) -> None:
        if self.h:
            lib.mynah_hip_sampler_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Qwen3Decoder:
    """The GPU decode state (include/mynah_decode.h) over a SynthQwen3."""

    def __init__(self, model: SynthQwen3, n_ctx: int):
        err = C.create_string_buffer(512)
        self.model = model
        self.h = lib.mynah_hip_qwen3_new(C.byref(model.c_shape), model.table, model.count,
                                         ptr(model.blob), model.blob.nbytes, n_ctx, err, 512)
        if not self.h:
            raise HipError(f"qwen3_new: {err.value.decode()}")

    @classmethod
    def from_gguf(cls, path: str, n_ctx: int = 0) -> "Qwen3Decoder":
        """The decoder over a GGUF checkpoint (mynah_slm_load, src/model.c:177):
        n_ctx 0, or above the file's context_length, takes context_length
        (src/arch_qwen3.c:94)."""
        with GgufFile(path, split=True) as g:
            shape, _ = g.qwen3_shape()
        self = cls.__new__(cls)
        self.model = types.SimpleNamespace(shape=shape, path=path)
        err = C.create_string_buffer(512)
        self.h = lib.mynah_hip_qwen3_from_gguf(os.fsencode(path), n_ctx, err, 512)
        if not self.h:
            raise HipError(f"qwen3_from_gguf: {err.value.decode(errors='replace')}")
        return self

    def read_attn(self) -> np.ndarray:
        """The last layer's attention output of the most recent step."""
        sh = self.model.shape
        out = np.empty(sh.n_heads * sh.head_dim, np.float32)
        check(lib.mynah_hip_qwen3_read_attn(self.h, ptr(out)), "read_attn")
        return out

    def set_kv(self, k: np.ndarray, v: np.ndarray, n_pos: int) -> None:
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        check(lib.mynah_hip_qwen3_set_kv(self.h, ptr(k), ptr(v), n_pos), "set_kv")

    def get_kv(self, n_pos: int):
        """Positions [0, n_pos) of the cache as (k, v), [layer][n_pos][kv_dim]."""
        sh = self.model.shape
        kv_dim = sh.n_kv_heads * sh.head_dim
        k = np.empty((sh.n_layers, n_pos, kv_dim), np.float32)
        v = np.empty_like(k)
        check(lib.mynah_hip_qwen3_get_kv(self.h, ptr(k), ptr(v), n_pos), "get_kv")
        return k, v

    def prefill(self, tokens) -> None:
        """Fill the cache with `tokens` at the next positions, no logits
        (bit-identical to one forward(token, want_logits=False) per token)."""
        p = np.ascontiguousarray(tokens, dtype=np.uint32)
        check(lib.mynah_hip_qwen3_prefill(self.h, ptr(p), p.size), "prefill")

    def set_prefill(self, mode: int) -> None:
        """PREFILL_BATCHED (default) or PREFILL_STEPS for prompt()."""
        check(lib.mynah_hip_qwen3_set_prefill(self.h, mode), "set_prefill")

    def forward(self, token: int, want_logits: bool = True):
        logits = np.empty(self.model.shape.vocab, np.float32) if want_logits else None
        check(lib.mynah_hip_qwen3_forward(self.h, token, ptr(logits) if want_logits else None),
              "forward")
        return logits

    def generate(self, first: int, steps: int):
        out = np.empty(steps, np.uint32)
        ms = C.c_float(0.0)
        check(lib.mynah_hip_qwen3_generate(self.h, first, steps, ptr(out), C.byref(ms)),
              "generate")
        return [int(t) for t in out], float(ms.value)

    def forced(self, inputs):
        """Teacher forcing through the replayed step graphs: step i runs
        inputs[i]; returns (greedy id of every step, last step's logits)."""
        p = np.ascontiguousarray(inputs, dtype=np.uint32)
        out = np.empty(p.size, np.uint32)
        logits = np.empty(self.model.shape.vocab, np.float32)
        check(lib.mynah_hip_qwen3_forced(self.h, ptr(p), p.size, ptr(out), ptr(logits)),
              "forced")
        return [int(t) for t in out], logits

    def generate_tokens(self, prompt, max_new: int, eos=(), sampler=None, chunk: int = 0,
                        stop_after=None, on_token=None, device_sampler=None):
        """The generation loop (include/mynah_generate.h). `sampler`: None for
        greedy on the device, else an object with a C handle `h` and
        `fn_addresses()` -> (sample, accept); `device_sampler`: a
        DeviceSampler, sampling inside the device steps instead (then
        `sampler` is unused). The token callback stops after
        `stop_after` ids, or when `on_token(id)` (if given) returns true.
        Returns (ids the callback saw, count the loop returned, timing)."""
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        e = np.ascontiguousarray(list(eos) or [0], dtype=np.uint32)
        seen = []

        def token_cb(_ctx, tok):
            seen.append(int(tok))
            if on_token is not None:
                return 1 if on_token(int(tok)) else 0
            return 1 if stop_after is not None and len(seen) >= stop_after else 0

        cb = TOKEN_FN(token_cb)
        gp = GenParams()
        gp.prompt, gp.n_prompt, gp.max_new = ptr(p), p.size, max_new
        gp.eos, gp.n_eos = ptr(e), len(eos)
        gp.on_token = C.cast(cb, C.c_void_p).value
        gp.chunk = chunk
        if device_sampler is not None:
            gp.device_sampler = device_sampler.h
        if sampler is not None:
            gp.sample, gp.accept = sampler.fn_addresses()
            gp.sampler = sampler.h
        t = GenTiming()
        n = lib.mynah_hip_qwen3_generate_tokens(self.h, C.byref(gp), C.byref(t))
        if n < 0:
            raise HipError(f"generate_tokens: {lib.mynah_hip_last_error().decode()}")
        return seen, int(n), t

    @property
    def n_past(self) -> int:
        return int(lib.mynah_hip_qwen3_n_past(self.h))

    def prompt(self, tokens, steps: int):
        """Prefill the prompt (all but its last token, no head), then `steps`
        greedy steps; returns (generated ids, prefill ms, decode ms)."""
        p = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.empty(steps, np.uint32)
        pm, dm = C.c_float(0.0), C.c_float(0.0)
        check(lib.mynah_hip_qwen3_prompt(self.h, ptr(p), p.size, steps, ptr(out), C.byref(pm),
                                         C.byref(dm)), "prompt")
        return [int(t) for t in out], float(pm.value), float(dm.value)

    def set_attention(self, mode: int) -> None:
        """ATTN_EXACT (the reference's order) or ATTN_SPLIT (positions split
        across workgroups, per-chunk softmax partials combined)."""
        check(lib.mynah_hip_qwen3_set_attention(self.h, mode), "set_attention")

    @property
    def uses_graph(self) -> bool:
        return bool(lib.mynah_hip_qwen3_uses_graph(self.h))

    def reset(self) -> None:
        lib.mynah_hip_qwen3_reset(self.h)

    def close(self) -> None:
        if self.h:
            lib.mynah_hip_qwen3_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def synth_uniform(seed: int, n: int, bound: int) -> np.ndarray:
    """n integers uniform in [0, bound) from the shared generator."""
    out = np.empty(n, np.uint32)
    check(lib.mynah_synth_uniform_u32(seed, n, bound, ptr(out)), "uniform")
    return out


def first_token(config_seed: int, vocab: int) -> int:
    """The first decode token of a config (uniform over the vocabulary)."""
    import configs
    return int(synth_uniform(substream(config_seed, configs.TOKEN_SEED_INDEX), 1, vocab)[0])
