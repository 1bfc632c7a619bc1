"""ctypes binding of libbsattn.so (the C ABI declared in include/bsattn.h).

Loading fails loudly when the library has not been built: there is no
fallback path.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# BSATTN_LIBRARY selects another build of the same C ABI (e.g. a tuning variant)
LIB_PATH = os.environ.get("BSATTN_LIBRARY") or os.path.join(HERE, "libbsattn.so")

OK = 0
ERR_INVALID = -1
ERR_HIP = -2
ERR_NO_PAGES = -3
ERR_RANGE = -4
ERR_NOMEM = -5
ERR_INTERNAL = -6

F16 = 0
BF16 = 1

# Every entry point declared in include/bsattn.h.
EXPORTS = (
    "bsattn_version",
    "bsattn_last_error",
    "bsattn_cache_create",
    "bsattn_cache_destroy",
    "bsattn_cache_info",
    "bsattn_shuffle_free_pages",
    "bsattn_seq_pages",
    "bsattn_seq_len",
    "bsattn_append",
    "bsattn_append_quantized",
    "bsattn_select",
    "bsattn_attend",
    "bsattn_decode",
    "bsattn_decode_noalloc",
    "bsattn_append_decode",
    "bsattn_decode_multi",
    "bsattn_prefill",
    "bsattn_reserve",
    "bsattn_append_step",
    "bsattn_sync",
    "bsattn_trim",
    "bsattn_reset",
    "bsattn_copy",
    "bsattn_export",
    "bsattn_export_quantized",
    "bsattn_export_summaries",
    "bsattn_profile_enable",
    "bsattn_profile_read",
)

KERNEL_SCORE, KERNEL_TOPK, KERNEL_ATTEND, KERNEL_COMBINE, KERNEL_APPEND, KERNEL_SUMMARY, KERNEL_PREFILL = range(7)


class BsattnError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"bsattn error {code}: {msg}")
        self.code = code


class Desc(ctypes.Structure):
    _fields_ = [
        ("max_seqs", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("kv_bits", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("top_k", ctypes.c_int32),
        ("sink_blocks", ctypes.c_int32),
        ("recent_blocks", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32),
        ("num_pages", ctypes.c_int64),
        ("device", ctypes.c_int32),
        ("reserved", ctypes.c_int32 * 3),
    ]


class Info(ctypes.Structure):
    _fields_ = [
        ("nsel_max", ctypes.c_int32),
        ("num_splits", ctypes.c_int32),
        ("page_bytes", ctypes.c_int64),
        ("pool_bytes", ctypes.c_int64),
        ("free_pages", ctypes.c_int64),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `make -C mlx-swift-lm_amd/csrc` "
            "(or __graft_entry__.build()); there is no fallback implementation")
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.c_void_p
    i32 = ctypes.c_int32
    PI32 = ctypes.POINTER(ctypes.c_int32)
    PP = ctypes.POINTER(ctypes.c_void_p)
    sig = {
        "bsattn_version": (i32, []),
        "bsattn_last_error": (ctypes.c_char_p, []),
        "bsattn_cache_create": (ctypes.c_int, [ctypes.POINTER(Desc), PP]),
        "bsattn_cache_destroy": (ctypes.c_int, [P]),
        "bsattn_cache_info": (ctypes.c_int, [P, ctypes.POINTER(Info)]),
        "bsattn_shuffle_free_pages": (ctypes.c_int, [P, ctypes.c_uint64]),
        "bsattn_seq_pages": (ctypes.c_int, [P, i32, PI32, i32, PI32]),
        "bsattn_seq_len": (ctypes.c_int, [P, i32, PI32]),
        "bsattn_append": (ctypes.c_int, [P, P, P, PI32, i32, i32, P]),
        "bsattn_append_quantized": (ctypes.c_int, [P, P, P, P, P, P, P, PI32, i32, i32, P]),
        "bsattn_select": (ctypes.c_int, [P, P, PI32, i32, P, P]),
        "bsattn_attend": (ctypes.c_int, [P, P, PI32, i32, P, ctypes.c_float, P, P]),
        "bsattn_decode": (ctypes.c_int, [P, P, PI32, i32, ctypes.c_float, P, P, P]),
        "bsattn_decode_noalloc": (ctypes.c_int, [P, P, PI32, i32, ctypes.c_float, P, P, P]),
        "bsattn_append_decode": (ctypes.c_int, [P, P, P, P, PI32, i32, ctypes.c_float, P, P, P]),
        "bsattn_decode_multi": (ctypes.c_int, [P, P, PI32, i32, i32, ctypes.c_float, P, P, P]),
        "bsattn_prefill": (ctypes.c_int, [P, P, PI32, i32, i32, ctypes.c_float, P, P]),
        "bsattn_reserve": (ctypes.c_int, [P, PI32, i32, i32, P]),
        "bsattn_append_step": (ctypes.c_int, [P, P, P, PI32, i32, P]),
        "bsattn_sync": (ctypes.c_int, [P, P]),
        "bsattn_trim": (ctypes.c_int, [P, PI32, i32, i32, PI32, P]),
        "bsattn_reset": (ctypes.c_int, [P, PI32, i32, P]),
        "bsattn_copy": (ctypes.c_int, [P, PP, P]),
        "bsattn_export": (ctypes.c_int, [P, PI32, i32, P, P, P]),
        "bsattn_export_quantized": (ctypes.c_int, [P, PI32, i32, P, P, P, P, P, P, P]),
        "bsattn_export_summaries": (ctypes.c_int, [P, i32, P, P]),
        "bsattn_profile_enable": (ctypes.c_int, [P, i32]),
        "bsattn_profile_read": (ctypes.c_int, [P, i32, ctypes.POINTER(ctypes.c_double),
                                               ctypes.POINTER(ctypes.c_int64)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != OK:
        msg = lib().bsattn_last_error()
        raise BsattnError(rc, msg.decode() if msg else "")


def i32_array(values):
    if values is None:
        return None
    arr = (ctypes.c_int32 * len(values))(*[int(v) for v in values])
    return arr
