"""libbsattn.so loads, exports every entry point include/bsattn.h declares,
and rejects bad arguments with status codes before touching the GPU.
CPU only: no call here reaches a HIP runtime function."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "bsattn.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bsattn_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import bsattn
    L = bsattn.lib()
    names = declared_symbols()
    assert len(names) >= 17
    for n in names:
        assert hasattr(L, n), f"{n} declared in bsattn.h but not exported"
    assert sorted(bsattn.EXPORTS) == names


def test_exports_are_c_linkage():
    out = os.popen(f"nm -D --defined-only {os.path.join(ROOT, 'mlx-swift-lm_amd', 'bsattn', 'libbsattn.so')}").read()
    for n in declared_symbols():
        assert re.search(rf"\bT {n}$", out, flags=re.M), f"{n} is not an unmangled text symbol"


def test_version_and_error_string():
    import bsattn
    L = bsattn.lib()
    assert L.bsattn_version() == 1
    assert isinstance(L.bsattn_last_error(), bytes)


def _desc(**kw):
    from bsattn import _lib
    base = dict(max_seqs=2, num_q_heads=32, num_kv_heads=8, head_dim=128, block_size=64,
                dtype=_lib.BF16, kv_bits=0, group_size=64, top_k=8, sink_blocks=1,
                recent_blocks=1, max_blocks_per_seq=16, num_pages=0, device=0)
    base.update(kw)
    return _lib.Desc(**base)


@pytest.mark.parametrize("bad,msg", [
    (dict(head_dim=64), "head_dim"),
    (dict(block_size=48), "block_size"),
    (dict(num_q_heads=30), "multiple"),
    (dict(num_q_heads=64, num_kv_heads=2), "GQA group"),
    (dict(recent_blocks=0), "recent_blocks"),
    (dict(dtype=7), "dtype"),
    (dict(max_blocks_per_seq=0), "max_blocks_per_seq"),
    (dict(max_seqs=0), "max_seqs"),
    (dict(kv_bits=3, dtype=0), "kv_bits"),
    (dict(kv_bits=4), "fp16"),
    (dict(kv_bits=8, dtype=0, group_size=32), "group_size"),
])
def test_create_rejects_bad_geometry(bad, msg):
    import bsattn
    L = bsattn.lib()
    h = ctypes.c_void_p()
    rc = L.bsattn_cache_create(ctypes.byref(_desc(**bad)), ctypes.byref(h))
    assert rc == -1
    assert msg in L.bsattn_last_error().decode()
    assert not h.value


def test_null_arguments_are_errors():
    import bsattn
    L = bsattn.lib()
    assert L.bsattn_cache_create(None, None) == -1
    assert L.bsattn_append(None, None, None, None, 1, 1, None) == -1
    assert L.bsattn_decode(None, None, None, 1, ctypes.c_float(1.0), None, None, None) == -1
    assert L.bsattn_decode_multi(None, None, None, 1, 2, ctypes.c_float(1.0), None, None, None) == -1
    assert L.bsattn_prefill(None, None, None, 1, 64, ctypes.c_float(1.0), None, None) == -1
    assert L.bsattn_reserve(None, None, 1, 1, None) == -1
    assert L.bsattn_append_step(None, None, None, None, 1, None) == -1
    assert L.bsattn_sync(None, None) == -1
    assert L.bsattn_select(None, None, None, 1, None, None) == -1
    assert L.bsattn_cache_info(None, None) == -1
    assert L.bsattn_append_quantized(None, None, None, None, None, None, None, None, 1, 1, None) == -1
    assert L.bsattn_export_quantized(None, None, 1, None, None, None, None, None, None, None) == -1
    assert L.bsattn_cache_destroy(None) == 0
