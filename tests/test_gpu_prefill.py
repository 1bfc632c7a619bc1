"""Dense causal prefill attention (bsattn_prefill): the last L tokens of
each sequence attend causally to everything before them, as the reference's
attentionWithCacheUpdate computes for L > 1 with the causal mask.  Every
query is checked against the oracle's dense attention over its prefix."""
from __future__ import annotations

import numpy as np
import pytest

from common import from_dev, log, make_workload, new_cache, output_error, to_dev, ulp
import oracle as O

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _run(w, gpu, L, pre_lens=None):
    """Caches holding each sequence minus its last L tokens, then the L
    tokens appended and prefilled; returns (out [B, Hq, L, D] bits, q)."""
    import torch
    c = new_cache(w)
    for b in range(w.B):
        T = w.lens[b]
        if T > L:
            c.append(to_dev(np.ascontiguousarray(w.keys[b][None, :, :T - L]), w.dtype, gpu),
                     to_dev(np.ascontiguousarray(w.values[b][None, :, :T - L]), w.dtype, gpu), seq_ids=[b])
    nk = np.stack([w.keys[b][:, w.lens[b] - L:] for b in range(w.B)])
    nv = np.stack([w.values[b][:, w.lens[b] - L:] for b in range(w.B)])
    c.append(to_dev(nk, w.dtype, gpu), to_dev(nv, w.dtype, gpu))
    qm = O.fill_normal(w.seed + 77, 0, 0, (w.B, w.Hq, L, w.D), w.dtype)
    out = c.prefill(to_dev(qm, w.dtype, gpu), w.scale)
    torch.cuda.synchronize()
    return from_dev(out), qm, c


def _check(w, got, qm, L, queries):
    worst = 0.0
    for b in range(w.B):
        for i in queries:
            pos = w.lens[b] - L + i
            for h in range(w.Hkv):
                ref = O.dense(qm[b, h * w.G:(h + 1) * w.G, i], w.keys[b][h][:pos + 1],
                              w.values[b][h][:pos + 1], w.scale, w.dtype)
                a = O.to_f32(got[b, h * w.G:(h + 1) * w.G, i], w.dtype).astype(np.float64)
                err = output_error(a, ref, w.dtype)
                assert err <= TOL, f"seq {b} query {i} head {h}: error {err:.3g}"
                worst = max(worst, err)
    return worst


@pytest.mark.parametrize("dtype,Hq,Hkv,Tb,lens,L", [
    ("bf16", 32, 8, 64, [3000, 2048], 100),
    ("f16", 32, 8, 32, [1500, 1999], 77),
    ("bf16", 64, 4, 64, [2600, 700], 64),     # G = 16: one query token per column set
    ("f16", 8, 8, 64, [1100, 900], 40),       # G = 1: 16 query tokens per column set
    ("bf16", 16, 2, 32, [640, 650], 33),      # G = 8
])
def test_prefill_matches_dense_attention(gpu, dtype, Hq, Hkv, Tb, lens, L):
    log(f"[prefill] {dtype} G={Hq // Hkv} Tb={Tb} L={L}")
    w = make_workload(7000 + Hq + Tb + L, B=len(lens), Hq=Hq, Hkv=Hkv, T=max(lens), Tb=Tb, dtype=dtype,
                      top_k=4, lens=lens, salient_frac=0.01)
    got, qm, _ = _run(w, gpu, L)
    err = _check(w, got, qm, L, sorted({0, 1, L // 2, L - 2, L - 1}))
    log(f"[prefill] err={err:.3g}")


def test_prefill_bf16_values_beyond_fp16(gpu):
    """bf16 V values fp16 cannot hold (|v| >= 65536, scaled by 2^17 on a few
    tokens): the units holding them take the bf16 PV path, the others the
    fp16 one; every checked query against the oracle."""
    log("[prefill] bf16 V beyond the fp16 range")
    L = 64
    w = make_workload(7700, B=2, Hq=32, Hkv=8, T=1500, Tb=64, dtype="bf16", top_k=4, lens=[1500, 1400])
    for b in range(w.B):
        v = O.to_f32(w.values[b], "bf16")
        rows = np.arange(37, w.lens[b], 211)          # a few tokens in several units
        v[:, rows, :] *= 2.0 ** 17
        w.values[b] = O.from_f32(v, "bf16")
    got, qm, _ = _run(w, gpu, L)
    # the error bound scales with sum_i p_i |v_i|, which the oracle's dense
    # attention over |V| gives; for unit-scale values it is the plain TOL
    worst = 0.0
    for b in range(w.B):
        for i in sorted({0, 1, L // 2, L - 1}):
            pos = w.lens[b] - L + i
            for h in range(w.Hkv):
                qh, kh, vh = qm[b, h * w.G:(h + 1) * w.G, i], w.keys[b][h][:pos + 1], w.values[b][h][:pos + 1]
                ref = O.dense(qh, kh, vh, w.scale, w.dtype)
                mag = O.dense(qh, kh, vh & np.uint16(0x7FFF), w.scale, w.dtype)
                a = O.to_f32(got[b, h * w.G:(h + 1) * w.G, i], w.dtype).astype(np.float64)
                err = float(np.max((np.abs(a - ref) - 0.5 * ulp(ref, w.dtype)) / np.maximum(1.0, mag)))
                assert err <= TOL, f"seq {b} query {i} head {h}: relative error {err:.3g}"
                worst = max(worst, err)
    log(f"[prefill] relative err={worst:.3g}")


def test_prefill_whole_prompt(gpu):
    """The whole prompt in one pass from an empty cache (L = T): every
    query checked, the first attends to itself only."""
    w = make_workload(7100, B=2, Hq=32, Hkv=8, T=300, Tb=64, dtype="bf16", top_k=2, lens=[300, 300])
    got, qm, c = _run(w, gpu, 300)
    assert c.offset == 300
    _check(w, got, qm, 300, range(0, 300, 7))
    # the first query attends to token 0 only: output = v[0]
    for b in range(w.B):
        for hq in range(w.Hq):
            assert np.array_equal(got[b, hq, 0], w.values[b][hq // w.G][0])


def test_attention_with_cache_update_prefill(gpu):
    import torch
    from bsattn import attentionWithCacheUpdate
    w = make_workload(7200, B=2, Hq=32, Hkv=8, T=500, Tb=64, dtype="bf16", top_k=2, lens=[500, 500])
    L = 40
    a = new_cache(w)
    b = new_cache(w)
    for c in (a, b):
        c.append(to_dev(np.stack([k[:, :460] for k in w.keys]), "bf16", gpu),
                 to_dev(np.stack([v[:, :460] for v in w.values]), "bf16", gpu))
    nk = to_dev(np.stack([k[:, 460:] for k in w.keys]), "bf16", gpu)
    nv = to_dev(np.stack([v[:, 460:] for v in w.values]), "bf16", gpu)
    q = to_dev(O.fill_normal(7201, 0, 0, (2, 32, L, 128), "bf16"), "bf16", gpu)
    o1 = attentionWithCacheUpdate(q, nk, nv, a, w.scale, mask="causal")
    b.append(nk, nv)
    o2 = b.prefill(q, w.scale)
    torch.cuda.synchronize()
    assert a.offset == 500 and torch.equal(o1, o2)


def test_prefill_argument_errors(gpu):
    import torch
    from bsattn import BsattnError
    w = make_workload(7300, B=1, Hq=32, Hkv=8, T=100, Tb=64, dtype="f16", top_k=2)
    c = new_cache(w)
    c.append(to_dev(w.keys[0][None], "f16", gpu), to_dev(w.values[0][None], "f16", gpu))
    with pytest.raises(BsattnError):
        c.prefill(torch.zeros((1, 32, 101, 128), dtype=torch.float16, device=gpu), 1.0)  # more queries than tokens


@pytest.mark.parametrize("bits,Hq,Hkv,Tb,lens,L", [
    (4, 32, 8, 64, [2000, 1300], 90),
    (8, 64, 4, 32, [1500, 800], 50),     # G = 16
    (8, 16, 8, 64, [700, 900], 33),      # G = 2
    (4, 32, 8, 32, [310, 97], 70),       # int4 in 32-token blocks; idle waves in the last workgroup
])
def test_prefill_quantized_cache(gpu, bits, Hq, Hkv, Tb, lens, L):
    """Prefill over an affine-quantized cache: each query against the
    oracle's attention over the quantized keys / values of its prefix."""
    import torch
    GS = 64
    log(f"[prefill-q] int{bits} G={Hq // Hkv} Tb={Tb} L={L}")
    w = make_workload(7400 + bits + Hq + L, B=len(lens), Hq=Hq, Hkv=Hkv, T=max(lens), Tb=Tb, dtype="f16",
                      top_k=4, lens=lens)
    c = new_cache(w, kv_bits=bits)
    for b in range(w.B):
        T = w.lens[b]
        c.append(to_dev(np.ascontiguousarray(w.keys[b][None, :, :T - L]), "f16", gpu),
                 to_dev(np.ascontiguousarray(w.values[b][None, :, :T - L]), "f16", gpu), seq_ids=[b])
    c.append(to_dev(np.stack([w.keys[b][:, w.lens[b] - L:] for b in range(w.B)]), "f16", gpu),
             to_dev(np.stack([w.values[b][:, w.lens[b] - L:] for b in range(w.B)]), "f16", gpu))
    qm = O.fill_normal(w.seed + 78, 0, 0, (w.B, w.Hq, L, w.D), "f16")
    got = from_dev(c.prefill(to_dev(qm, "f16", gpu), w.scale))
    torch.cuda.synchronize()
    worst = 0.0
    for b in range(w.B):
        kq = [O.quantize(w.keys[b][h], bits, GS) for h in range(w.Hkv)]
        vq = [O.quantize(w.values[b][h], bits, GS) for h in range(w.Hkv)]
        for i in sorted({0, 1, L // 2, L - 1}):
            pos = w.lens[b] - L + i
            idx = np.arange(pos // Tb + 1, dtype=np.int32)
            for h in range(w.Hkv):
                ref = O.attend_q(qm[b, h * w.G:(h + 1) * w.G, i], [a[:pos + 1] for a in kq[h]],
                                 [a[:pos + 1] for a in vq[h]], Tb, bits, GS, idx, w.scale)
                a = O.to_f32(got[b, h * w.G:(h + 1) * w.G, i], "f16").astype(np.float64)
                err = output_error(a, ref, "f16")
                assert err <= 1e-2, f"seq {b} query {i} head {h}: error {err:.3g}"
                worst = max(worst, err)
    log(f"[prefill-q] err={worst:.3g}")


def _threads():
    import os
    return max(1, min(16, len(os.sched_getaffinity(0))))


@pytest.mark.parametrize("bits", [0, 4])
def test_prefill_timed_shape(gpu, bits):
    """The benchmarked prefill shape: a 512-token chunk appended at the end of
    32768 tokens, B=8, Hq=32, Hkv=8, 64-token blocks (bf16, or an int4 affine
    cache over fp16 inputs).  Every head of every sequence at the first and
    last 8 query tokens and at two middle ones, against the oracle's attention
    over the query's prefix (dense, or over the quantized keys / values);
    the oracle calls run on a thread pool (ctypes releases the GIL)."""
    import torch
    from concurrent.futures import ThreadPoolExecutor
    B, Hq, Hkv, Tb, T, L, GS = 8, 32, 8, 64, 32768, 512, 64
    dtype = "bf16" if bits == 0 else "f16"
    log(f"[prefill-timed] {'bf16' if bits == 0 else 'int4'}: generating")
    w = make_workload(7800 + bits, B=B, Hq=Hq, Hkv=Hkv, T=T, Tb=Tb, dtype=dtype, top_k=32, salient_frac=0.01)
    c = new_cache(w, kv_bits=bits)
    for b in range(B):
        c.append(to_dev(np.ascontiguousarray(w.keys[b][None, :, :T - L]), dtype, gpu),
                 to_dev(np.ascontiguousarray(w.values[b][None, :, :T - L]), dtype, gpu), seq_ids=[b])
    c.append(to_dev(np.stack([w.keys[b][:, T - L:] for b in range(B)]), dtype, gpu),
             to_dev(np.stack([w.values[b][:, T - L:] for b in range(B)]), dtype, gpu))
    qm = O.fill_normal(7850 + bits, 0, 0, (B, Hq, L, w.D), dtype)
    got = from_dev(c.prefill(to_dev(qm, dtype, gpu), w.scale))
    torch.cuda.synchronize()
    queries = list(range(8)) + [L // 3, 2 * L // 3] + list(range(L - 8, L))
    log(f"[prefill-timed] checking {B * Hkv * len(queries)} (sequence, kv head, query) triples")

    def job(item):
        b, h, i = item
        pos = T - L + i
        qh = np.ascontiguousarray(qm[b, h * w.G:(h + 1) * w.G, i])
        if bits == 0:
            ref = O.dense(qh, w.keys[b][h][:pos + 1], w.values[b][h][:pos + 1], w.scale, dtype)
        else:
            kq, vq = qcache[(b, h)]
            ref = O.attend_q(qh, [a[:pos + 1] for a in kq], [a[:pos + 1] for a in vq], Tb, bits, GS,
                             np.arange(pos // Tb + 1, dtype=np.int32), w.scale)
        a = O.to_f32(got[b, h * w.G:(h + 1) * w.G, i], dtype).astype(np.float64)
        return output_error(a, ref, dtype)

    qcache = {}
    if bits:
        with ThreadPoolExecutor(_threads()) as ex:
            pairs = [(b, h) for b in range(B) for h in range(Hkv)]
            codes = ex.map(lambda p: (O.quantize(w.keys[p[0]][p[1]], bits, GS),
                                      O.quantize(w.values[p[0]][p[1]], bits, GS)), pairs)
            qcache = dict(zip(pairs, codes))
    with ThreadPoolExecutor(_threads()) as ex:
        errs = list(ex.map(job, [(b, h, i) for b in range(B) for h in range(Hkv) for i in queries]))
    worst = max(errs)
    log(f"[prefill-timed] max error {worst:.3g}")
    assert worst <= (TOL if bits == 0 else 1e-2), f"max error {worst:.3g}"


def _random_prefill(seed: int):
    r = np.random.default_rng(7900 + seed)
    bits = int(r.choice([0, 0, 4, 8]))
    dtype = "f16" if bits else str(r.choice(["f16", "bf16"]))
    G = int(r.choice([1, 2, 4, 8, 16]))
    Hkv = int(r.choice([1, 2, 4])) if G >= 8 else int(r.choice([1, 2, 4, 8]))
    Tb = int(r.choice([32, 64]))
    L = int(r.integers(17, 401))
    # a whole prompt from an empty cache (16-bit caches) or a chunk after earlier tokens
    lens = [L + int(r.choice([0 if bits == 0 else 1, int(r.integers(1, 3000))]))
            for _ in range(int(r.integers(1, 4)))]
    return bits, dtype, Hkv * G, Hkv, Tb, lens, L


@pytest.mark.parametrize("seed", range(12))
def test_prefill_random(gpu, seed):
    """Seeded random shapes: cache type (fp16, bf16, int4, int8), GQA group,
    block size, 17 - 400 query tokens, ragged lengths (some the whole prompt
    from an empty cache); the first, second, middle and last two queries of
    every head against the oracle's attention over the query's prefix."""
    bits, dtype, Hq, Hkv, Tb, lens, L = _random_prefill(seed)
    log(f"[prefill random {seed}] bits={bits} {dtype} Hq={Hq} Hkv={Hkv} Tb={Tb} lens={lens} L={L}")
    if bits:
        test_prefill_quantized_cache(gpu, bits, Hq, Hkv, Tb, lens, L)
        return
    w = make_workload(7950 + seed, B=len(lens), Hq=Hq, Hkv=Hkv, T=max(lens), Tb=Tb, dtype=dtype,
                      top_k=4, lens=lens, salient_frac=0.01)
    got, qm, _ = _run(w, gpu, L)
    err = _check(w, got, qm, L, sorted({0, 1, L // 2, L - 2, L - 1}))
    log(f"[prefill random {seed}] err={err:.3g}")
