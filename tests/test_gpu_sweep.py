"""Every attention kernel instantiation the dispatch can launch: 16-bit
(fp16, bf16) and affine-quantized (int4, int8) caches x 32- and 64-token
blocks x GQA groups 1, 2, 4, 8, 16, at small ragged sizes (a partial last
block, two sequences of different lengths).  For each: selection bit-exact
with the oracle, decode (selection fused into the attention) bit-identical
to select + attend (given indices), and both within the bars of the parity
and quantized suites.  The kernels differ per (Tb, G, bits) in register
allocation and instruction scheduling, so each combination is run once.
"""
from __future__ import annotations

import pytest

from common import fill, log, make_workload, new_cache
from test_gpu_parity import run_and_check
from test_gpu_quant import quantize_all, run_and_check_q

pytestmark = pytest.mark.gpu

GROUPS = [1, 2, 4, 8, 16]


def _workload(seed, dtype, Tb, G):
    lens = [20 * Tb + 7, 9 * Tb]
    return make_workload(seed, B=len(lens), Hq=2 * G, Hkv=2, T=max(lens), Tb=Tb, dtype=dtype, top_k=6,
                         ns=1, nr=1, lens=lens, salient_frac=0.02)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("Tb", [32, 64])
@pytest.mark.parametrize("G", GROUPS)
def test_sweep_16bit(gpu, dtype, Tb, G):
    log(f"[sweep] {dtype} Tb={Tb} G={G}")
    w = _workload(4100 + Tb + G, dtype, Tb, G)
    cache = new_cache(w)
    fill(cache, w, gpu)
    run_and_check(cache, w, gpu)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("Tb", [32, 64])
@pytest.mark.parametrize("G", GROUPS)
def test_sweep_quantized(gpu, bits, Tb, G):
    log(f"[sweep] int{bits} Tb={Tb} G={G}")
    w = _workload(4200 + bits + Tb + G, "f16", Tb, G)
    cache = new_cache(w, kv_bits=bits)
    fill(cache, w, gpu)
    kq, vq = quantize_all(w, bits)
    run_and_check_q(cache, w, gpu, bits, kq, vq)
