"""Seeded random shapes against the oracle: cache type (fp16, bf16, int4 and
int8 affine), block size, GQA group, batch, ragged lengths (some shorter than
one block), top_k (from one block to more than a sequence's candidates), and
sink and recent counts.  Each shape runs the path the dispatch picks for it
(the selection fused into the attention, the block-wide selection, MFMA
scoring with the exact band, the split-combine variants) and is held to the
parity bars: selection bit-exact, decode identical to select + attend,
outputs within 2e-3 of the oracle."""
from __future__ import annotations

import numpy as np
import pytest

from common import fill, log, make_workload, new_cache
from test_gpu_parity import run_and_check
from test_gpu_quant import quantize_all, run_and_check_q

pytestmark = pytest.mark.gpu

KINDS = ["f16", "bf16", "int4", "int8"]


def shape(seed: int) -> dict:
    r = np.random.default_rng(9000 + seed)
    Tb = int(r.choice([32, 64]))
    G = int(r.choice([1, 2, 4, 8, 16]))
    Hkv = int(r.choice([1, 2, 4])) if G >= 8 else int(r.choice([1, 2, 4, 8]))
    B = int(r.integers(1, 4))
    nb_max = 2100 if seed % 5 == 0 else 600
    lens = [int(r.integers(1, nb_max * Tb)) for _ in range(B)]
    if seed % 3 == 0 and B > 1:
        lens[0] = int(r.integers(1, Tb))  # shorter than one block
    return dict(kind=KINDS[seed % 4], Tb=Tb, G=G, Hkv=Hkv, lens=lens,
                top_k=int(r.choice([1, 2, 5, 17, 32, 64, 100, 130, 250])),
                ns=int(r.integers(0, 3)), nr=int(r.choice([1, 2, 4])),
                salient=float(r.choice([0.0, 0.01, 0.02])))


@pytest.mark.parametrize("seed", range(48))
def test_random_shape(gpu, seed):
    s = shape(seed)
    log(f"[random {seed}] {s}")
    bits = {"int4": 4, "int8": 8}.get(s["kind"], 0)
    dtype = "f16" if bits else s["kind"]
    w = make_workload(9100 + seed, B=len(s["lens"]), Hq=s["Hkv"] * s["G"], Hkv=s["Hkv"], T=max(s["lens"]),
                      Tb=s["Tb"], dtype=dtype, top_k=s["top_k"], ns=s["ns"], nr=s["nr"], lens=s["lens"],
                      salient_frac=s["salient"])
    cache = new_cache(w, kv_bits=bits) if bits else new_cache(w)
    fill(cache, w, gpu)
    if bits:
        kq, vq = quantize_all(w, bits)
        err = run_and_check_q(cache, w, gpu, bits, kq, vq)
    else:
        err = run_and_check(cache, w, gpu)
    log(f"[random {seed}] err={err:.3g}")
