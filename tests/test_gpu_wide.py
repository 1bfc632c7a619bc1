"""Nine-wave attention workgroups.  A call whose selected blocks fill every
CU with one workgroup of 9 waves takes them instead of 4-wave workgroups
(attend_waves in csrc/bsattn_kernels.hip): 2 sequences x 8 kv heads with 130
selected blocks are 16 pairs x 15 splits = 240 workgroups, where 4 waves
would make 528, 3 on some CUs.  Quantized caches with groups of 16 heads and
32-token blocks may take two such workgroups per CU (4 sequences x 8 kv
heads: 480 workgroups, 18 waves on the busiest CU against 20).  Each shape here has more than 256 candidates
per sequence, so the decode runs the scoring kernel and the attention kernel
with the selection inside (not the one-launch fused decode), and is held to
the parity bars: selection bit-exact, decode == select + attend, outputs
against the oracle, for every cache type (fp16, bf16, int4, int8), both
block sizes and groups of 1, 2 and 4 heads; then a multi-token decode
against its single-token decodes (both take the same splits: the wave count
follows the call's sequences, not a launch's entries)."""
from __future__ import annotations

import numpy as np
import pytest

from common import fill, log, make_workload, new_cache
from test_gpu_multi import test_multi_decode_equals_sequential_decodes as multi_check
from test_gpu_parity import run_and_check
from test_gpu_quant import quantize_all, run_and_check_q

pytestmark = pytest.mark.gpu

WIDE, BASE, MAX_BATCH = 9, 4, 64


def takes_wide(Hkv: int, G: int, nsel: int, nseq: int, cus: int, bits: int = 0, Tb: int = 64) -> bool:
    """The library's choice of 9-wave workgroups, restated: groups of up to 4
    heads with at most one workgroup per CU, or quantized groups of 16 heads
    in 32-token blocks with at most two; and fewer waves on the busiest CU
    than 4-wave workgroups spread over the CUs would leave."""
    two = bits != 0 and G == 16 and Tb == 32
    if G > 4 and not two:
        return False
    pairs = min(max(nseq, 1), MAX_BATCH) * Hkv
    per_cu = -(-pairs * -(-nsel // WIDE) // cus)
    if per_cu > (2 if two else 1):
        return False
    base = pairs * -(-nsel // BASE)
    return WIDE * per_cu < BASE * -(-base // cus)


def cus() -> int:
    import torch
    return torch.cuda.get_device_properties(0).multi_processor_count


# kind, Tb, G, lengths (more than 256 candidates each)
CASES = {
    "bf16-tb64-g4": ("bf16", 64, 4, [340 * 64 - 5, 300 * 64 + 17]),
    "f16-tb64-g4": ("f16", 64, 4, [330 * 64 + 1, 290 * 64 + 40]),
    "f16-tb32-g2": ("f16", 32, 2, [320 * 32 - 1, 280 * 32 + 9]),
    "bf16-tb32-g1": ("bf16", 32, 1, [300 * 32 + 3, 297 * 32]),
    "int4-tb64-g4": ("int4", 64, 4, [310 * 64 - 7, 290 * 64 + 30]),
    "int4-tb32-g2": ("int4", 32, 2, [330 * 32 + 5, 270 * 32 + 2]),
    "int8-tb64-g1": ("int8", 64, 1, [300 * 64 + 11, 285 * 64]),
    "int8-tb32-g4": ("int8", 32, 4, [340 * 32 - 3, 310 * 32 + 1]),
    # 16-head groups: one workgroup per CU, then two
    "int8-tb32-g16": ("int8", 32, 16, [330 * 32 + 7, 290 * 32 - 1]),
    "int8-tb32-g16-two": ("int8", 32, 16, [300 * 32 + 1, 320 * 32 - 5, 280 * 32 + 16, 340 * 32]),
}
HKV, TOP_K = 8, 128


@pytest.mark.parametrize("case", list(CASES))
def test_wide_workgroups_against_the_oracle(gpu, case):
    kind, Tb, G, lens = CASES[case]
    bits = {"int4": 4, "int8": 8}.get(kind, 0)
    dtype = "f16" if bits else kind
    w = make_workload(9700 + len(case) + Tb + G, B=len(lens), Hq=HKV * G, Hkv=HKV, T=max(lens), Tb=Tb,
                      dtype=dtype, top_k=TOP_K, ns=1, nr=1, lens=lens, salient_frac=0.01)
    assert takes_wide(HKV, G, w.nsel_max, w.B, cus(), bits, Tb), "shape does not take the 9-wave workgroups"
    log(f"[wide] {case}: {w.B} x {HKV} pairs, {w.nsel_max} slots, {-(-w.nsel_max // WIDE)} splits")
    cache = new_cache(w, kv_bits=bits) if bits else new_cache(w)
    fill(cache, w, gpu)
    if bits:
        kq, vq = quantize_all(w, bits)
        err = run_and_check_q(cache, w, gpu, bits, kq, vq)
    else:
        err = run_and_check(cache, w, gpu)
    log(f"[wide] {case} err={err:.3g}")


# dtype, Tb, Hq, Hkv, K, L, kv_bits, lens: the multi-token decode's checks
# (bit-identical to L single decodes, each query against the oracle on its
# prefix for 16-bit caches) at shapes that take the 9-wave workgroups
MULTI = {
    "bf16-tb64-g4-l3": ("bf16", 64, 32, 8, 127, 3, 0, [320 * 64 + 2, 300 * 64 + 1]),
    "f16-tb32-g2-l4": ("f16", 32, 16, 8, 127, 4, 0, [300 * 32 + 3, 310 * 32 + 1]),
    "int8-tb64-g4-l2": ("f16", 64, 32, 8, 127, 2, 8, [300 * 64 + 9, 280 * 64]),
    "int8-tb32-g16-l2": ("f16", 32, 128, 8, 127, 2, 8, [300 * 32 + 5, 280 * 32 + 3]),
}


@pytest.mark.parametrize("case", list(MULTI))
def test_wide_multi_decode_equals_single_decodes(gpu, case):
    dtype, Tb, Hq, Hkv, K, L, bits, lens = MULTI[case]
    # the multi-token test's caches keep 1 sink and 2 recent blocks
    assert takes_wide(Hkv, Hq // Hkv, K + 3, len(lens), cus(), bits, Tb)
    log(f"[wide multi] {case}")
    multi_check(gpu, dtype, Hq, Hkv, Tb, K, L, bits, lens)
