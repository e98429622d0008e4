"""TEST INFRASTRUCTURE ONLY: ctypes access to the CPU oracle (liboracle.so)
and, where it was built, to the reference's own host sources
(oracle/_ref/libdlref.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.  The product package never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
sz = C.c_size_t


class Dims(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("q_heads", C.c_uint32), ("kv_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("ffn", C.c_uint32), ("vocab", C.c_uint32),
                ("eps", C.c_float), ("theta", C.c_double)]


class Block(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("input_norm", "wq", "wk", "wv", "q_norm", "k_norm",
                                          "wo", "post_norm", "wg", "wu", "wd")]


class MT64(C.Structure):
    _fields_ = [("words", C.c_uint64 * 312), ("index", C.c_uint32)]


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = C.CDLL(path)
        L.or_bf16_from_f32.argtypes = [C.c_float]
        L.or_bf16_from_f32.restype = C.c_uint16
        L.or_f32_from_bf16.argtypes = [C.c_uint16]
        L.or_f32_from_bf16.restype = C.c_float
        for name in ("orc_projection", "ors_projection"):
            getattr(L, name).argtypes = [u16p, u16p, u16p, sz, sz, sz]
        for name in ("orc_rms_norm", "ors_rms_norm"):
            getattr(L, name).argtypes = [u16p, u16p, u16p, sz, sz, C.c_float]
        for name in ("orc_rotary", "ors_rotary"):
            getattr(L, name).argtypes = [u16p, u16p, sz, sz, sz, sz, C.c_double]
        for name in ("orc_attention", "ors_attention"):
            getattr(L, name).argtypes = [u16p, u16p, u16p, u16p, sz, sz, sz, sz, sz, sz, sz]
        L.orc_rms_inverse.argtypes = [u16p, sz, C.c_float]
        L.orc_rms_inverse.restype = C.c_float
        L.orc_attention_scale.argtypes = [sz]
        L.orc_attention_scale.restype = C.c_float
        L.orc_add.argtypes = [u16p, u16p, u16p, sz]
        L.orc_steer.argtypes = [u16p, f32p, sz]
        for name in ("orc_silu_multiply", "ors_silu_multiply"):
            getattr(L, name).argtypes = [u16p, u16p, u16p, sz]
        L.orc_embedding.argtypes = [u32p, u16p, u16p, sz, sz]
        L.orc_qwen3_block_forward.argtypes = [C.POINTER(Dims), C.POINTER(Block), u16p, sz, sz,
                                              u16p, u16p]
        L.orc_qwen3_logits.argtypes = [C.POINTER(Dims), u16p, u16p, u16p, u16p]
        L.orc_greedy_bf16.argtypes = [u16p, sz, C.POINTER(C.c_uint32)]
        L.orc_inject.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, sz, C.c_float, f32p]
        L.orc_inject.restype = C.c_uint32
        L.orc_direction.argtypes = [C.c_void_p, C.c_void_p, C.c_int, sz, f32p]
        L.orc_direction.restype = C.c_uint32
        L.orc_intervene.argtypes = [C.c_void_p, C.c_int, sz, sz, f32p, sz, sz, C.c_float, u32p]
        L.orc_intervene.restype = C.c_int
        L.orc_greedy_bf16.restype = C.c_int
        L.or_mt64_seed.argtypes = [C.POINTER(MT64), C.c_uint64]
        L.or_mt64_next.argtypes = [C.POINTER(MT64)]
        L.or_mt64_next.restype = C.c_uint64
        L.ors_categorical_select.argtypes = [f32p, sz, C.c_int, C.c_double, sz, C.c_double,
                                             C.POINTER(MT64), C.POINTER(C.c_uint32)]
        L.ors_categorical_select.restype = C.c_int
        L.ors_categorical_select_bits.argtypes = [f32p, sz, C.c_int, C.c_double, sz, C.c_double,
                                                  C.c_uint64, C.POINTER(C.c_uint32)]
        L.ors_categorical_select_bits.restype = C.c_int
        L.ors_categorical_select_bits_exp.argtypes = [f32p, sz, C.c_int, C.c_double, sz, C.c_double,
                                                      C.c_uint64, C.c_int, C.POINTER(C.c_uint32)]
        L.ors_categorical_select_bits_exp.restype = C.c_int
        f64o = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
        L.ors_categorical_trace.argtypes = [f32p, sz, C.c_double, sz, C.c_double, C.c_int, u32p, f64o,
                                            f64o, C.POINTER(sz), C.POINTER(sz)]
        L.ors_categorical_trace.restype = C.c_int
        L.or_fill_normal_bf16.argtypes = [u16p, sz, C.c_uint64, C.c_uint64, C.c_float, sz]
        L.or_set_threads.argtypes = [C.c_int]
        L.orc_rope_angles.argtypes = [sz, sz, C.c_double, f32p, f32p]
        f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
        L.or_math_exp.argtypes = [f64p, f64p, sz]
        L.or_math_expf.argtypes = [f32p, f32p, sz]
        L.or_math_log.argtypes = [f64p, f64p, sz]
        L.or_math_sincos.argtypes = [f64p, f64p, f64p, sz]
        L.or_math_pow.argtypes = [f64p, f64p, f64p, sz]
        _LIB = L
    return _LIB


def ref():
    """The reference's own categorical sampler/BF16 code, or None when
    oracle/_ref was not built (it needs /root/reference at build time)."""
    global _REF
    if _REF is None:
        path = os.path.join(HERE, "_ref", "libdlref.so")
        if not os.path.exists(path):
            return None
        R = C.CDLL(path)
        R.dlref_categorical_select.argtypes = [f32p, sz, C.c_int, C.c_double, sz, C.c_double,
                                               C.c_uint64, C.c_uint32, u32p]
        R.dlref_categorical_select.restype = C.c_int
        R.dlref_mt64.argtypes = [C.c_uint64, C.c_uint64]
        R.dlref_mt64.restype = C.c_uint64
        R.dlref_bf16_from_f32.argtypes = [C.c_float]
        R.dlref_bf16_from_f32.restype = C.c_uint16
        R.dlref_f32_from_bf16.argtypes = [C.c_uint16]
        R.dlref_f32_from_bf16.restype = C.c_float
        _REF = R
    return _REF


# ---------------------------------------------------------------- helpers
def bf16_from_f32(a: np.ndarray) -> np.ndarray:
    """Vectorised RNE narrowing with NaN -> 0x7fc0 (bf16.cpp:48-55)."""
    bits = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    nan = (bits & 0x7FFFFFFF) > 0x7F800000
    out = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    out[nan] = 0x7FC0
    return out


def f32_from_bf16(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def operand(count: int, seed: int) -> np.ndarray:
    """tests/gpu/operator_reference.cpp:60-75: ((i*73 + seed*37) mod 257 - 128)/64,
    rounded to BF16."""
    i = np.arange(count, dtype=np.int64)
    v = (((i * 73 + seed * 37) % 257) - 128).astype(np.float32) / np.float32(64)
    return bf16_from_f32(v)


def normal_bf16(n: int, seed: int, stream: int, scale: float, first: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().or_fill_normal_bf16(out, n, seed, stream, scale, first)
    return out


def projection(x, w, rows, in_w, out_w, serial=False):
    y = np.empty(rows * out_w, dtype=np.uint16)
    (lib().ors_projection if serial else lib().orc_projection)(
        np.ascontiguousarray(x, np.uint16), np.ascontiguousarray(w, np.uint16), y, rows, in_w, out_w)
    return y


def rms_norm(x, w, rows, width, eps, serial=False):
    y = np.empty(rows * width, dtype=np.uint16)
    (lib().ors_rms_norm if serial else lib().orc_rms_norm)(
        np.ascontiguousarray(x, np.uint16), np.ascontiguousarray(w, np.uint16), y, rows, width, eps)
    return y


def rotary(x, positions, heads, width, first, theta, serial=False):
    y = np.empty(positions * heads * width, dtype=np.uint16)
    (lib().ors_rotary if serial else lib().orc_rotary)(
        np.ascontiguousarray(x, np.uint16), y, positions, heads, width, first, theta)
    return y


def attention(q, k, v, positions, q_heads, kv_heads, width, first, pos_stride=None,
              head_stride=None, serial=False):
    if pos_stride is None:
        pos_stride = kv_heads * width
    if head_stride is None:
        head_stride = width
    y = np.empty(positions * q_heads * width, dtype=np.uint16)
    (lib().ors_attention if serial else lib().orc_attention)(
        np.ascontiguousarray(q, np.uint16), np.ascontiguousarray(k, np.uint16),
        np.ascontiguousarray(v, np.uint16), y, positions, q_heads, kv_heads, width, first,
        pos_stride, head_stride)
    return y


def add(a, b):
    y = np.empty(len(a), dtype=np.uint16)
    lib().orc_add(np.ascontiguousarray(a, np.uint16), np.ascontiguousarray(b, np.uint16), y, len(a))
    return y


def steer(h: np.ndarray, vector: np.ndarray) -> None:
    """In place: h <- BF16(FP32(h) + vector)."""
    lib().orc_steer(h, np.ascontiguousarray(vector, np.float32), len(h))


def silu_multiply(g, u, serial=False):
    y = np.empty(len(g), dtype=np.uint16)
    (lib().ors_silu_multiply if serial else lib().orc_silu_multiply)(
        np.ascontiguousarray(g, np.uint16), np.ascontiguousarray(u, np.uint16), y, len(g))
    return y


def _typed(a, bf16):
    return np.ascontiguousarray(a, np.uint16 if bf16 else np.float32)


def inject(source, source_bf16: bool, output_bf16: bool, scale: float):
    """orc_inject (injection.cu:49-98): returns (status, norm, output); the
    output holds zeros where the oracle wrote nothing."""
    src = _typed(source, source_bf16)
    out = np.zeros(src.size, dtype=np.uint16 if output_bf16 else np.float32)
    norm = np.zeros(1, np.float32)
    status = lib().orc_inject(src.ctypes.data, int(source_bf16), out.ctypes.data, int(output_bf16), src.size,
                              scale, norm)
    return int(status), float(norm[0]), out


def direction(original, edited, bf16: bool):
    """orc_direction (steering.cu:69-100): returns (status, FP32 direction)."""
    a, b = _typed(original, bf16), _typed(edited, bf16)
    out = np.zeros(a.size, dtype=np.float32)
    status = lib().orc_direction(a.ctypes.data, b.ctypes.data, int(bf16), a.size, out)
    return int(status), out


def intervene(residual, bf16: bool, rows: int, width: int, u, first: int, selected: int, strength: float, state):
    """orc_intervene (steering.cu:107-159) in place on `residual` and `state`
    (uint32[2]); returns whether the chunk held the selected row."""
    assert residual.dtype == (np.uint16 if bf16 else np.float32) and residual.flags.c_contiguous
    return bool(lib().orc_intervene(residual.ctypes.data, int(bf16), rows, width,
                                    np.ascontiguousarray(u, np.float32), first, selected, strength, state))


def greedy(logits_bf16) -> tuple[int, int]:
    out = C.c_uint32(0)
    status = lib().orc_greedy_bf16(np.ascontiguousarray(logits_bf16, np.uint16), len(logits_bf16),
                                   C.byref(out))
    return status, out.value


def categorical_bits(logits_f32, mode, temperature, top_k, top_p, bits) -> tuple[int, int]:
    out = C.c_uint32(0)
    status = lib().ors_categorical_select_bits(np.ascontiguousarray(logits_f32, np.float32),
                                               len(logits_f32), mode, temperature, top_k, top_p,
                                               bits, C.byref(out))
    return status, out.value


def categorical_bits_exp(logits_f32, mode, temperature, top_k, top_p, bits, build_exp) -> tuple[int, int]:
    """The law with the weight exp chosen: build_exp False = glibc exp (the
    reference host), True = the build's dl_exp (the device's serial replay)."""
    out = C.c_uint32(0)
    status = lib().ors_categorical_select_bits_exp(np.ascontiguousarray(logits_f32, np.float32),
                                                   len(logits_f32), mode, temperature, top_k, top_p,
                                                   bits, int(build_exp), C.byref(out))
    return status, out.value


def categorical_trace(logits_f32, temperature, top_k, top_p, build_exp=False):
    """Serial quantities of the categorical law: (ids in kept order, F_k for
    k = 1..size, G_i for i = 1..cutoff)."""
    x = np.ascontiguousarray(logits_f32, np.float32)
    n = len(x)
    ids = np.zeros(n, np.uint32)
    fold = np.zeros(n, np.float64)
    cumulative = np.zeros(n, np.float64)
    size, count = C.c_size_t(0), C.c_size_t(0)
    status = lib().ors_categorical_trace(x, n, temperature, top_k, top_p, int(build_exp), ids, fold,
                                         cumulative, C.byref(size), C.byref(count))
    assert status == 0, status
    return ids[: size.value], fold[: size.value], cumulative[: count.value]


class MT19937_64:
    def __init__(self, seed: int):
        self.state = MT64()
        lib().or_mt64_seed(C.byref(self.state), seed)

    def __call__(self) -> int:
        return lib().or_mt64_next(C.byref(self.state))


class Qwen3Weights:
    """Row-major BF16 weights of a Qwen3 model, as numpy arrays, in the
    reference's parameter layout (W[O, I])."""

    def __init__(self, dims: Dims, blocks: list[dict], final_norm, lm_head, embedding):
        self.dims = dims
        self.blocks = blocks
        self.final_norm = final_norm
        self.lm_head = lm_head
        self.embedding = embedding

    def block_struct(self, i: int) -> Block:
        b = self.blocks[i]
        return Block(*[b[n].ctypes.data for n in ("input_norm", "wq", "wk", "wv", "q_norm", "k_norm",
                                                   "wo", "post_norm", "wg", "wu", "wd")])


def block_forward(weights: Qwen3Weights, layer: int, h: np.ndarray, rows: int, first: int,
                  k_cache: np.ndarray, v_cache: np.ndarray) -> None:
    blk = weights.block_struct(layer)
    lib().orc_qwen3_block_forward(C.byref(weights.dims), C.byref(blk), h, rows, first, k_cache,
                                  v_cache)


def logits(weights: Qwen3Weights, h_row: np.ndarray) -> np.ndarray:
    out = np.empty(weights.dims.vocab, dtype=np.uint16)
    lib().orc_qwen3_logits(C.byref(weights.dims), weights.final_norm, weights.lm_head,
                           np.ascontiguousarray(h_row, np.uint16), out)
    return out
