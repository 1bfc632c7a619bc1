"""ctypes binding of the CPU oracle (libbsattn_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker.  The product library never
imports it.

Arrays are numpy; fp16/bf16 tensors travel as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbsattn_oracle.so")

F16, BF16 = 0, 1
DTYPE_CODE = {"f16": F16, "fp16": F16, "float16": F16, "bf16": BF16, "bfloat16": BF16}

_lib = None


def build(force: bool = False) -> str:
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "-B" if force else "all"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i32, i64, u64, f64 = ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_double
        sig = {
            "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f64_to_f16": (ctypes.c_uint16, [f64]),
            "orc_f64_to_bf16": (ctypes.c_uint16, [f64]),
            "orc_to_f32": (None, [P, i64, i32, P]),
            "orc_from_f32": (None, [P, i64, i32, P]),
            "orc_splitmix64": (u64, [u64]),
            "orc_hash3": (u64, [u64, u64, u64]),
            "orc_normal": (f64, [u64, u64, u64]),
            "orc_fill_normal": (None, [u64, u64, u64, i64, i64, P, i32, P]),
            "orc_choose_positions": (None, [u64, u64, u64, i32, i32, P]),
            "orc_uniform_int": (i64, [u64, u64, u64, i64, i64]),
            "orc_block_summary": (None, [P, i64, i32, i32, i32, P]),
            "orc_summaries": (i32, [P, i32, i32, i32, i32, P]),
            "orc_affine_params": (None, [P, i32, i32, P, P]),
            "orc_quantize_affine": (None, [P, i64, i32, i32, i32, P, P, P]),
            "orc_dequantize_affine": (None, [P, P, P, i64, i32, i32, i32, P]),
            "orc_block_summary_q": (None, [P, P, P, i32, i32, i32, i32, P]),
            "orc_summaries_q": (i32, [P, P, P, i32, i32, i32, i32, i32, P]),
            "orc_dot_canonical": (ctypes.c_float, [P, P, i32, i32]),
            "orc_score_blocks": (None, [P, i32, P, i32, i32, i32, P]),
            "orc_score_key": (ctypes.c_uint32, [ctypes.c_float]),
            "orc_select": (i32, [P, i32, i32, i32, i32, i32, P]),
            "orc_attend": (None, [P, i32, P, P, i32, i32, i32, P, i32, f64, i32, P]),
            "orc_attend_q": (None, [P, i32, P, P, P, P, P, P, i32, i32, i32, i32, i32, P, i32, f64, P]),
            "orc_dense": (None, [P, i32, P, P, i32, i32, f64, i32, P]),
            "orc_block_mass": (None, [P, P, i32, i32, i32, f64, P]),
            "orc_decode_head": (i32, [P, i32, P, P, i32, i32, i32, i32, i32, i32, f64, i32, P, P]),
            "orc_omp_threads": (i32, []),
            "orc_layer_step": (None, [P] * 10 + [i32] * 11 + [f64, i32, P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def dcode(dtype) -> int:
    return DTYPE_CODE[dtype] if isinstance(dtype, str) else int(dtype)


# ---- numeric formats -------------------------------------------------------

def to_f32(bits: np.ndarray, dtype) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().orc_to_f32(_p(bits), bits.size, dcode(dtype), _p(out))
    return out


def from_f32(x: np.ndarray, dtype) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_from_f32(_p(x), x.size, dcode(dtype), _p(out))
    return out


# ---- RNG -------------------------------------------------------------------

def fill_normal(seed: int, stream: int, start: int, shape, dtype, row_mult=None) -> np.ndarray:
    """out.flat[i] = round_dtype(normal(seed, stream, start + i) * row_mult[i // row_len])
    where row_len = shape[-1]."""
    out = np.empty(shape, np.uint16)
    n = out.size
    row_len = shape[-1] if len(shape) else 1
    rm = None
    if row_mult is not None:
        rm = np.ascontiguousarray(row_mult, dtype=np.float64)
        assert rm.size == n // row_len
    lib().orc_fill_normal(seed, stream, start, n, row_len, _p(rm) if rm is not None else None,
                          dcode(dtype), _p(out))
    return out


def choose_positions(seed: int, stream: int, key: int, n: int, count: int) -> np.ndarray:
    out = np.empty(count, np.int32)
    lib().orc_choose_positions(seed, stream, key, n, count, _p(out))
    return out


def uniform_int(seed: int, stream: int, index: int, lo: int, hi: int) -> int:
    return int(lib().orc_uniform_int(seed, stream, index, lo, hi))


# ---- summaries / scoring / selection ---------------------------------------

def summaries(keys: np.ndarray, Tb: int, dtype) -> np.ndarray:
    """keys [T, D] uint16 -> summaries of full blocks [T // Tb, D]."""
    keys = np.ascontiguousarray(keys, np.uint16)
    T, D = keys.shape
    out = np.empty((max(T // Tb, 0), D), np.uint16)
    lib().orc_summaries(_p(keys), T, D, Tb, dcode(dtype), _p(out))
    return out


def summaries_q(codes, scales, biases, Tb: int, bits: int, gs: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, np.uint32)
    scales = np.ascontiguousarray(scales, np.uint16)
    biases = np.ascontiguousarray(biases, np.uint16)
    T = codes.shape[0]
    D = codes.shape[1] * 32 // bits
    out = np.empty((T // Tb, D), np.uint16)
    lib().orc_summaries_q(_p(codes), _p(scales), _p(biases), T, D, Tb, bits, gs, _p(out))
    return out


def dot_canonical(a: np.ndarray, b: np.ndarray, dtype) -> float:
    a = np.ascontiguousarray(a, np.uint16)
    b = np.ascontiguousarray(b, np.uint16)
    return float(lib().orc_dot_canonical(_p(a), _p(b), a.size, dcode(dtype)))


def score_blocks(q: np.ndarray, summ: np.ndarray, dtype) -> np.ndarray:
    """q [G, D], summ [n, D] -> scores [n] fp32."""
    q = np.ascontiguousarray(q, np.uint16)
    summ = np.ascontiguousarray(summ, np.uint16)
    G, D = q.shape
    n = summ.shape[0]
    out = np.empty(n, np.float32)
    lib().orc_score_blocks(_p(q), G, _p(summ), n, D, dcode(dtype), _p(out))
    return out


def score_key(s: float) -> int:
    return int(lib().orc_score_key(s))


def select(scores: np.ndarray, length: int, Tb: int, ns: int, nr: int, K: int):
    nb = -(-length // Tb)
    sc = np.zeros(max(nb, 1), np.float32)
    scores = np.asarray(scores, np.float32)
    sc[: min(len(scores), len(sc))] = scores[: len(sc)]
    out = np.empty(ns + nr + K, np.int32)
    n = lib().orc_select(_p(sc), length, Tb, ns, nr, K, _p(out))
    return out, int(n)


# ---- attention -------------------------------------------------------------

def attend(q, keys, values, Tb: int, idx, scale: float, dtype) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint16)
    keys = np.ascontiguousarray(keys, np.uint16)
    values = np.ascontiguousarray(values, np.uint16)
    idx = np.ascontiguousarray(idx, np.int32)
    G, D = q.shape
    T = keys.shape[0]
    out = np.empty((G, D), np.float64)
    lib().orc_attend(_p(q), G, _p(keys), _p(values), T, D, Tb, _p(idx), idx.size, scale,
                     dcode(dtype), _p(out))
    return out


def attend_q(q, kq, vq, Tb: int, bits: int, gs: int, idx, scale: float) -> np.ndarray:
    """kq / vq = (codes [T, D*bits/32] u32, scales [T, D/gs] f16, biases [T, D/gs] f16)."""
    q = np.ascontiguousarray(q, np.uint16)
    kc, ks, kb = (np.ascontiguousarray(a) for a in kq)
    vc, vs, vb = (np.ascontiguousarray(a) for a in vq)
    idx = np.ascontiguousarray(idx, np.int32)
    G, D = q.shape
    T = kc.shape[0]
    out = np.empty((G, D), np.float64)
    lib().orc_attend_q(_p(q), G, _p(kc), _p(ks), _p(kb), _p(vc), _p(vs), _p(vb), T, D, Tb, bits,
                       gs, _p(idx), idx.size, scale, _p(out))
    return out


def dense(q, keys, values, scale: float, dtype) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint16)
    keys = np.ascontiguousarray(keys, np.uint16)
    values = np.ascontiguousarray(values, np.uint16)
    G, D = q.shape
    out = np.empty((G, D), np.float64)
    lib().orc_dense(_p(q), G, _p(keys), _p(values), keys.shape[0], D, scale, dcode(dtype), _p(out))
    return out


def block_mass(q_f16, keys_f32, Tb: int, scale: float) -> np.ndarray:
    q_f16 = np.ascontiguousarray(q_f16, np.uint16)
    keys_f32 = np.ascontiguousarray(keys_f32, np.float32)
    T, D = keys_f32.shape
    out = np.empty(-(-T // Tb), np.float64)
    lib().orc_block_mass(_p(q_f16), _p(keys_f32), T, D, Tb, scale, _p(out))
    return out


def decode_head(q, keys, values, Tb, ns, nr, K, scale, dtype):
    """One (sequence, kv-head): summary -> score -> select -> attend."""
    q = np.ascontiguousarray(q, np.uint16)
    keys = np.ascontiguousarray(keys, np.uint16)
    values = np.ascontiguousarray(values, np.uint16)
    G, D = q.shape
    T = keys.shape[0]
    idx = np.empty(ns + nr + K, np.int32)
    out = np.empty((G, D), np.float64)
    n = lib().orc_decode_head(_p(q), G, _p(keys), _p(values), T, D, Tb, ns, nr, K, scale,
                              dcode(dtype), _p(idx), _p(out))
    return idx, int(n), out


# ---- MLX affine codec -------------------------------------------------------

def affine_params(x_f32: np.ndarray, bits: int):
    """fp32 (scale, bias) of one group, before their fp16 cast."""
    x = np.ascontiguousarray(x_f32, np.float32)
    s = np.zeros(1, np.float32)
    b = np.zeros(1, np.float32)
    lib().orc_affine_params(_p(x), x.size, bits, _p(s), _p(b))
    return float(s[0]), float(b[0])


def quantize(x_f16: np.ndarray, bits: int, gs: int):
    x = np.ascontiguousarray(x_f16, np.uint16)
    D = x.shape[-1]
    rows = x.size // D
    codes = np.empty(x.shape[:-1] + (D * bits // 32,), np.uint32)
    scales = np.empty(x.shape[:-1] + (D // gs,), np.uint16)
    biases = np.empty(x.shape[:-1] + (D // gs,), np.uint16)
    lib().orc_quantize_affine(_p(x), rows, D, bits, gs, _p(codes), _p(scales), _p(biases))
    return codes, scales, biases


def dequantize(codes, scales, biases, bits: int, gs: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, np.uint32)
    scales = np.ascontiguousarray(scales, np.uint16)
    biases = np.ascontiguousarray(biases, np.uint16)
    D = codes.shape[-1] * 32 // bits
    rows = codes.size // codes.shape[-1]
    out = np.empty(codes.shape[:-1] + (D,), np.float32)
    lib().orc_dequantize_affine(_p(codes), _p(scales), _p(biases), rows, D, bits, gs, _p(out))
    return out


def layer_step(q, summ, Tb, ns, nr, K, scale, dtype, keys=None, values=None, kq=None, vq=None,
               bits=0, gs=64):
    """One decode layer-step of every (sequence, kv head) given the block
    summaries, OpenMP-parallel over the pairs.  q [B, Hq, D]; summ
    [B, Hkv, T/Tb, D]; 16-bit keys / values [B, Hkv, T, D], or quantized
    kq / vq = (codes [B, Hkv, T, W], scales, biases [B, Hkv, T, D/gs]).
    -> (idx [B, Hkv, ns+nr+K] int32, out [B, Hq, D] float64)."""
    q = np.ascontiguousarray(q, np.uint16)
    summ = np.ascontiguousarray(summ, np.uint16)
    B, Hq, D = q.shape
    Hkv = summ.shape[1]
    if bits:
        kq = tuple(np.ascontiguousarray(a) for a in kq)
        vq = tuple(np.ascontiguousarray(a) for a in vq)
        T = kq[0].shape[2]
        ptrs = [None, None, _p(kq[0]), _p(kq[1]), _p(kq[2]), _p(vq[0]), _p(vq[1]), _p(vq[2])]
    else:
        keys = np.ascontiguousarray(keys, np.uint16)
        values = np.ascontiguousarray(values, np.uint16)
        T = keys.shape[2]
        ptrs = [_p(keys), _p(values)] + [None] * 6
    idx = np.empty((B, Hkv, ns + nr + K), np.int32)
    out = np.empty((B, Hq, D), np.float64)
    lib().orc_layer_step(_p(q), _p(summ), *ptrs, B, Hq, Hkv, T, D, Tb, bits, gs, ns, nr, K, scale,
                         dcode(dtype), _p(idx), _p(out))
    return idx, out


def omp_threads() -> int:
    return int(lib().orc_omp_threads())
