"""The fused decode kernel (scoring, selection, gather + attention in one
launch, one workgroup per (entry, kv head) split) against the CPU oracle,
through the C ABI: selected blocks bit-exact, outputs within 2e-3 (net of
the final rounding), decode bit-identical to select + attend (the given-index
mode of the same kernel).  Covers one split per pair with several gather
rounds per wave (batches of >= 256 (entry, kv head) pairs), the multi-split
plan with few candidates, both block sizes and dtypes, GQA groups 1 / 2 / 4,
both summary-load orders (all rows at once, or the length first for ragged
batches), blocks past a partial tail, and top_k = 0 (sinks and recent only)
on every selection path."""
from __future__ import annotations

import numpy as np
import pytest

from common import (fill, from_dev, log, make_workload, new_cache, oracle_decode, oracle_summaries,
                    output_error, to_dev)
import oracle as O

pytestmark = pytest.mark.gpu

TOL = 2e-3


def check_decode(cache, w, device, summaries=True):
    import torch
    q = to_dev(w.q[:, :, None, :], w.dtype, device)
    idx_ref, out_ref = oracle_decode(w)
    out = cache.decode(q, w.scale)
    idx = cache.selectBlocks(q)
    out2 = cache.attend(q, idx, w.scale)
    torch.cuda.synchronize()
    idx = idx.cpu().numpy()
    assert np.array_equal(idx, idx_ref), f"selected blocks differ: {np.argwhere(idx != idx_ref)[:5]}"
    a = from_dev(out).reshape(w.B, w.Hq, w.D)
    assert np.array_equal(a, from_dev(out2).reshape(w.B, w.Hq, w.D)), "decode != select + attend"
    err = output_error(O.to_f32(a, w.dtype).astype(np.float64), out_ref, w.dtype)
    assert err <= TOL, f"output error {err:.3g} > {TOL}"
    if summaries:
        for b in range(w.B):
            assert np.array_equal(from_dev(cache.exportSummaries(b)), oracle_summaries(w, b))
    return err


@pytest.mark.parametrize("dtype,Tb,Hq,Hkv", [
    ("bf16", 64, 16, 4), ("f16", 64, 16, 4), ("f16", 32, 16, 8), ("bf16", 32, 8, 8), ("bf16", 64, 16, 8),
])
def test_single_split_rounds_ragged(gpu, dtype, Tb, Hq, Hkv):
    """>= 256 pairs: one workgroup per (entry, kv head), every wave gathering
    several blocks (online softmax across rounds); ragged lengths (partial
    tails, fewer candidates than top_k, a one-token sequence) make the host
    pick the length-first summary loads."""
    B = 256 // Hkv
    rng = np.random.default_rng(9100 + Tb + Hq)
    lens = [int(x) for x in rng.integers(1, 40 * Tb, B)]
    lens[0], lens[1], lens[2] = 1, Tb, 3 * Tb + 1
    log(f"[fused-rounds] {dtype} Tb={Tb} Hq={Hq} Hkv={Hkv} B={B}")
    w = make_workload(9100 + Tb + Hq, B=B, Hq=Hq, Hkv=Hkv, T=max(lens), Tb=Tb, dtype=dtype, top_k=20,
                      ns=1, nr=2, lens=lens)
    cache = new_cache(w)
    fill(cache, w, gpu, chunk=5 * Tb + 3)
    err = check_decode(cache, w, gpu, summaries=False)
    for b in (0, 3, B - 1):
        assert np.array_equal(from_dev(cache.exportSummaries(b)), oracle_summaries(w, b))
    log(f"[fused-rounds] err={err:.3g}")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_single_split_uniform_rows(gpu, dtype):
    """>= 256 pairs whose rows fill the block table: every summary row is
    loaded before the length is known and the first two chunks are scored
    without waiting for it."""
    Tb, Hkv, B = 64, 8, 32
    T = 24 * Tb - 5
    log(f"[fused-uniform] {dtype}")
    w = make_workload(9200, B=B, Hq=32, Hkv=Hkv, T=T, Tb=Tb, dtype=dtype, top_k=8, salient_frac=0.01)
    cache = new_cache(w, mbps=(T + Tb - 1) // Tb)
    fill(cache, w, gpu)
    check_decode(cache, w, gpu, summaries=False)


@pytest.mark.parametrize("dtype,Tb", [("f16", 64), ("bf16", 32)])
def test_multi_split_few_candidates(gpu, dtype, Tb):
    """A small batch (several splits per pair, each scoring the pair's few
    candidates itself), including the decode of config 1's shape."""
    log(f"[fused-multisplit] {dtype} Tb={Tb}")
    w = make_workload(9300 + Tb, B=2, Hq=32, Hkv=8, T=4096, Tb=Tb, dtype=dtype, top_k=8,
                      lens=[4096, 2500])
    cache = new_cache(w)
    fill(cache, w, gpu, chunk=700)
    check_decode(cache, w, gpu)


@pytest.mark.parametrize("Hq,Hkv,T", [
    (32, 8, 64 * 40 + 9),      # fused decode, few candidates
    (32, 8, 64 * 600),         # selection inside the attention kernel (many candidates, several splits)
    (64, 4, 64 * 1100),        # GQA 16, > 1024 candidates: MFMA scores + workgroup selection kernel
])
def test_top_k_zero_keeps_sinks_and_recent(gpu, Hq, Hkv, T):
    """top_k = 0 with candidates present: only the sink and recent blocks are
    attended (no ranking), on every selection path."""
    log(f"[topk0] Hq={Hq} Hkv={Hkv} T={T}")
    w = make_workload(9400 + Hq, B=2, Hq=Hq, Hkv=Hkv, T=T, Tb=64, dtype="bf16", top_k=0, ns=2, nr=3,
                      lens=[T, T - 70])
    cache = new_cache(w)
    fill(cache, w, gpu)
    check_decode(cache, w, gpu, summaries=False)
    import torch
    idx = cache.selectBlocks(to_dev(w.q[:, :, None, :], "bf16", gpu)).cpu().numpy()
    nb = -(-w.lens[1] // 64)
    assert idx[1, 0].tolist() == [0, 1, nb - 3, nb - 2, nb - 1]


def test_append_decode_single_split_loop(gpu):
    """The one-call decode step on >= 256 pairs (append launch, then the fused
    kernel) equals append then decode bit for bit across block fills, and
    matches the oracle at the end."""
    import torch
    Tb, Hkv, B, STEPS = 64, 8, 32, 70
    rng = np.random.default_rng(9500)
    lens = [int(x) for x in rng.integers(Tb, 12 * Tb, B)]
    w = make_workload(9500, B=B, Hq=32, Hkv=Hkv, T=max(lens) + STEPS, Tb=Tb, dtype="f16", top_k=6,
                      lens=[n + STEPS for n in lens])
    a, b = new_cache(w), new_cache(w)
    for c in (a, b):
        for s in range(B):
            c.append(to_dev(np.ascontiguousarray(w.keys[s][None, :, :lens[s]]), "f16", gpu),
                     to_dev(np.ascontiguousarray(w.values[s][None, :, :lens[s]]), "f16", gpu), seq_ids=[s])
    g = torch.Generator(device=gpu)
    g.manual_seed(9501)
    for i in range(STEPS):
        k = torch.stack([torch.from_numpy(w.keys[s][:, lens[s] + i].view(np.int16)) for s in range(B)])
        v = torch.stack([torch.from_numpy(w.values[s][:, lens[s] + i].view(np.int16)) for s in range(B)])
        k = k.to(gpu).view(torch.float16)[:, :, None, :].contiguous()
        v = v.to(gpu).view(torch.float16)[:, :, None, :].contiguous()
        q = torch.randn(B, 32, 1, 128, device=gpu, generator=g).half()
        o1 = a.appendDecode(k, v, q, w.scale)
        b.append(k, v)
        o2 = b.decode(q, w.scale)
        torch.cuda.synchronize()
        assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), f"step {i}"
    check_decode(a, w, gpu, summaries=False)
