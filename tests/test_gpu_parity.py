"""HIP path vs the CPU oracle, through the C ABI (libbsattn.so via ctypes).

Bars:
  * block summaries and selected block indices: bit-exact;
  * attention outputs: max-abs error <= 2e-3 against the fp64 oracle, net of
    the final rounding of the output to fp16/bf16 (|gpu - ref| - ulp(ref)/2).
"""
from __future__ import annotations

import math
import sys

import numpy as np
import pytest

from common import (S_LEN, Workload, check_config_inputs, check_literal_bar, config_args, fill, from_dev, log,
                    make_workload, new_cache, oracle_decode, oracle_summaries, output_error, to_dev, torch_dtype)
import oracle as O

pytestmark = pytest.mark.gpu

TOL = 2e-3


def run_and_check(cache, w: Workload, device, check_summaries=True):
    import torch
    q = to_dev(w.q[:, :, None, :], w.dtype, device)
    idx_ref, out_ref = oracle_decode(w)
    idx = cache.selectBlocks(q)
    out = cache.attend(q, idx, w.scale)
    out2 = cache.decode(q, w.scale)
    torch.cuda.synchronize()
    idx = idx.cpu().numpy()
    assert np.array_equal(idx, idx_ref), f"selected blocks differ: {np.argwhere(idx != idx_ref)[:5]}"
    got = O.to_f32(from_dev(out).reshape(w.B, w.Hq, w.D), w.dtype).astype(np.float64)
    got2 = from_dev(out2).reshape(w.B, w.Hq, w.D)
    assert np.array_equal(from_dev(out).reshape(w.B, w.Hq, w.D), got2), "decode != select + attend"
    err = output_error(got, out_ref, w.dtype)
    assert err <= TOL, f"output error {err:.3g} > {TOL}"
    check_literal_bar(got, out_ref, w.dtype, TOL, f"B{w.B} Hq{w.Hq} T{max(w.lens)} {w.dtype}")
    if check_summaries:
        for b in range(w.B):
            s = from_dev(cache.exportSummaries(b))
            assert np.array_equal(s, oracle_summaries(w, b)), f"summaries differ for seq {b}"
    return err


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_config1_single_decode(gpu, dtype):
    """B=1, Hq=32, Hkv=8, D=128, 4096 tokens in 64-token blocks, top-8 + sink + newest."""
    log(f"[config1] dtype={dtype}")
    w = make_workload(**config_args(f"C1_{dtype}"))
    check_config_inputs(w, f"C1_{dtype}")
    cache = new_cache(w)
    fill(cache, w, gpu)
    err = run_and_check(cache, w, gpu)
    log(f"[config1] dtype={dtype} err={err:.3g}")


def test_config2_batched_salient(gpu):
    """B=8, 32k context, bf16, 1% of keys scaled x8, top-32 + sink + recent."""
    log("[config2] generating")
    w = make_workload(**config_args("C2"))
    check_config_inputs(w, "C2")
    cache = new_cache(w)
    fill(cache, w, gpu)
    err = run_and_check(cache, w, gpu)
    log(f"[config2] err={err:.3g}")


@pytest.mark.parametrize("dtype,Tb,Hq,Hkv", [
    ("f16", 64, 32, 8), ("bf16", 64, 32, 8), ("f16", 32, 32, 8), ("bf16", 32, 64, 4),
    ("f16", 64, 16, 16), ("bf16", 64, 16, 8), ("f16", 32, 16, 2),
])
def test_ragged_paged(gpu, dtype, Tb, Hq, Hkv):
    """Ragged lengths (partial last blocks, shorter than one block, fewer
    candidates than top_k) with interleaved page order."""
    lens = [1, Tb - 1, Tb, Tb + 1, 7 * Tb + 5, 40 * Tb + 17, 23 * Tb]
    log(f"[ragged] {dtype} Tb={Tb} Hq={Hq} Hkv={Hkv}")
    w = make_workload(2000 + Tb + Hq, B=len(lens), Hq=Hq, Hkv=Hkv, T=max(lens), Tb=Tb,
                      dtype=dtype, top_k=6, ns=2, nr=2, lens=lens)
    cache = new_cache(w)
    fill(cache, w, gpu, chunk=3 * Tb + 7)
    run_and_check(cache, w, gpu)


@pytest.mark.parametrize("K,dtype", [(26, "f16"), (58, "bf16"), (110, "f16"), (170, "bf16"), (230, "f16"),
                                     (300, "bf16")])
def test_split_combine_variants(gpu, K, dtype):
    """top_k + sink + newest = 4 x splits: 7, 15, 28, 43, 58 and 76 splits, one
    per combine variant (up to 8 and 16 splits with every (m, l) in each
    thread, up to 32, 48 and 64 with the weights shared through LDS, the loop
    beyond); ragged lengths leave the last split of the shorter sequence
    partly empty."""
    Tb = 32
    lens = [Tb * 700 - 5, Tb * (K + 40)]
    log(f"[combine] K={K} splits={(K + 2 + 3) // 4} {dtype}")
    w = make_workload(3050 + K, B=2, Hq=32, Hkv=8, T=max(lens), Tb=Tb, dtype=dtype, top_k=K, lens=lens)
    cache = new_cache(w)
    fill(cache, w, gpu)
    err = run_and_check(cache, w, gpu)
    log(f"[combine] K={K} err={err:.3g}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_topk_covering_all_blocks_is_dense(gpu, dtype):
    """top_k >= number of blocks -> every block is attended and the result is
    dense decode attention (the reference's path, AttentionUtils.swift:68-75)."""
    w = make_workload(3000, B=2, Hq=32, Hkv=8, T=1000, Tb=64, dtype=dtype, top_k=64)
    cache = new_cache(w)
    fill(cache, w, gpu)
    run_and_check(cache, w, gpu)
    import torch
    q = to_dev(w.q[:, :, None, :], w.dtype, gpu)
    out = O.to_f32(from_dev(cache.decode(q, w.scale)).reshape(w.B, w.Hq, w.D), dtype)
    for b in range(w.B):
        for h in range(w.Hkv):
            ref = O.dense(w.q[b, h * 4:(h + 1) * 4], w.keys[b][h], w.values[b][h], w.scale, dtype)
            assert output_error(out[b, h * 4:(h + 1) * 4].astype(np.float64), ref, dtype) <= TOL


def test_ties_break_to_lower_index(gpu):
    """Every full block of a sequence has the same keys -> equal scores ->
    the lowest-index candidates are kept."""
    w = make_workload(3100, B=2, Hq=32, Hkv=8, T=20 * 64 + 9, Tb=64, dtype="bf16", top_k=5)
    for b in range(w.B):
        for h in range(w.Hkv):
            blk = w.keys[b][h][:64].copy()
            for j in range(w.lens[b] // 64):
                w.keys[b][h][j * 64:(j + 1) * 64] = blk
    cache = new_cache(w)
    fill(cache, w, gpu)
    run_and_check(cache, w, gpu)
    q = to_dev(w.q[:, :, None, :], w.dtype, gpu)
    idx = cache.selectBlocks(q).cpu().numpy()
    nb = -(-w.lens[0] // 64)
    assert list(idx[0, 0]) == [0, 1, 2, 3, 4, 5, nb - 1]


def test_decode_loop_with_appends(gpu):
    """Variable-length sequences; each step appends one token per sequence
    (crossing block boundaries, summaries refreshed on fill), then
    select + attend; every step checked against the oracle."""
    import torch
    Tb, steps = 64, 70
    lens0 = [100, 130, 190, 64]
    total = [l + steps for l in lens0]
    w = make_workload(3200, B=4, Hq=32, Hkv=8, T=max(total), Tb=Tb, dtype="f16", top_k=2,
                      lens=total)
    cache = new_cache(w)
    for b in range(w.B):
        k = np.ascontiguousarray(w.keys[b][:, :lens0[b]][None])
        v = np.ascontiguousarray(w.values[b][:, :lens0[b]][None])
        cache.append(to_dev(k, "f16", gpu), to_dev(v, "f16", gpu), seq_ids=[b])
    worst = 0.0
    for s in range(steps):
        cur = [l + s + 1 for l in lens0]
        k = np.stack([w.keys[b][:, cur[b] - 1:cur[b]] for b in range(w.B)])
        v = np.stack([w.values[b][:, cur[b] - 1:cur[b]] for b in range(w.B)])
        cache.append(to_dev(k, "f16", gpu), to_dev(v, "f16", gpu))
        ws = Workload(w.seed, w.B, w.Hq, w.Hkv, w.D, Tb, "f16", cur, w.top_k, w.ns, w.nr)
        ws.q = w.q
        ws.keys = [w.keys[b][:, :cur[b]] for b in range(w.B)]
        ws.values = [w.values[b][:, :cur[b]] for b in range(w.B)]
        worst = max(worst, run_and_check(cache, ws, gpu, check_summaries=(s % 10 == 9)))
    log(f"[decode-loop] worst err={worst:.3g}")


def test_config4_decode_loop_full(gpu):
    """B=32 sequences of U[8192, 65536] tokens (stream 4), their pages taken
    in shuffled physical order (the free list permuted from the seed, stream
    5), Hq=32, Hkv=8, fp16, top-32 + sink + recent; 256 decode steps, each
    appending one token per sequence: selected blocks and outputs against the
    oracle after steps 1, 128 and 256 (every head), block summaries after the
    last."""
    import torch
    seed, steps, Tb = 1004, 256, 64
    lens0 = [O.uniform_int(seed, S_LEN, b, 8192, 65536) for b in range(32)]
    total = [l + steps for l in lens0]
    log("[config4] generating")
    w = make_workload(**config_args("C4"))
    assert w.lens == total and w.seed == seed and w.Tb == Tb
    check_config_inputs(w, "C4")

    def view(cur):
        ws = Workload(w.seed, w.B, w.Hq, w.Hkv, w.D, Tb, "f16", list(cur), w.top_k, w.ns, w.nr)
        ws.q = w.q
        ws.keys = [w.keys[b][:, :cur[b]] for b in range(w.B)]
        ws.values = [w.values[b][:, :cur[b]] for b in range(w.B)]
        return ws

    cache = new_cache(w)
    cache.shuffleFreePages(seed)
    fill(cache, view(lens0), gpu)
    # the pages of a sequence are scattered through the pool, not ascending
    bt = cache.seqPages(0)
    assert bt != sorted(bt) and len(set(bt)) == len(bt)
    worst = 0.0
    for s in range(steps):
        cur = [l + s + 1 for l in lens0]
        k = np.stack([w.keys[b][:, cur[b] - 1:cur[b]] for b in range(w.B)])
        v = np.stack([w.values[b][:, cur[b] - 1:cur[b]] for b in range(w.B)])
        cache.append(to_dev(k, "f16", gpu), to_dev(v, "f16", gpu))
        if s + 1 in (1, 128, steps):
            log(f"[config4] step {s + 1}")
            worst = max(worst, run_and_check(cache, view(cur), gpu, check_summaries=(s + 1 == steps)))
    torch.cuda.synchronize()
    log(f"[config4] worst err={worst:.3g}")


def test_cache_contract_export_copy_trim(gpu):
    """Structural contract of the reference's KVCacheTests
    (Tests/MLXLMTests/KVCacheTests.swift:15-180): state round trip, copy()
    independence, trim semantics."""
    import torch
    w = make_workload(3300, B=2, Hq=32, Hkv=8, T=300, Tb=64, dtype="bf16", top_k=2)
    cache = new_cache(w, mbps=16)
    fill(cache, w, gpu)
    k, v = cache.state
    assert tuple(k.shape) == (2, 8, 300, 128)
    assert np.array_equal(from_dev(k), np.stack(w.keys))
    assert np.array_equal(from_dev(v), np.stack(w.values))
    assert cache.offset == 300 and cache.metaState[4] == "300"
    # copy is independent
    c2 = cache.copy()
    extra = to_dev(np.stack(w.keys)[:, :, :5], "bf16", gpu)
    c2.append(extra, extra)
    assert c2.offset == 305 and cache.offset == 300
    k1, _ = cache.state
    assert np.array_equal(from_dev(k1), np.stack(w.keys))
    # trim: back to 300 - 40 tokens then re-append the same 40 -> same results as before
    assert cache.trim(40) == 40 and cache.offset == 260
    tail_k = np.ascontiguousarray(np.stack(w.keys)[:, :, 260:])
    tail_v = np.ascontiguousarray(np.stack(w.values)[:, :, 260:])
    cache.append(to_dev(tail_k, "bf16", gpu), to_dev(tail_v, "bf16", gpu))
    run_and_check(cache, w, gpu)
    # trim clamps at the length
    assert cache.trim(10_000) == 300 and cache.offset == 0
    # state setter restores
    cache.state = [k, v]
    run_and_check(cache, w, gpu)
    # reset returns every page
    free_before = cache.freePages
    cache.reset([0, 1])
    assert cache.freePages == free_before + 2 * 5


def test_attention_with_cache_update(gpu):
    """attentionWithCacheUpdate: append the new token, then block-sparse decode."""
    from bsattn import attentionWithCacheUpdate
    T = 700
    w = make_workload(3400, B=3, Hq=32, Hkv=8, T=T + 1, Tb=64, dtype="bf16", top_k=4)
    cache = new_cache(w)
    for b in range(w.B):
        cache.append(to_dev(w.keys[b][None, :, :T], "bf16", gpu),
                     to_dev(w.values[b][None, :, :T], "bf16", gpu), seq_ids=[b])
    newk = np.ascontiguousarray(np.stack([w.keys[b][:, T:] for b in range(w.B)]))
    newv = np.ascontiguousarray(np.stack([w.values[b][:, T:] for b in range(w.B)]))
    q = to_dev(w.q[:, :, None, :], "bf16", gpu)
    out = attentionWithCacheUpdate(q, to_dev(newk, "bf16", gpu), to_dev(newv, "bf16", gpu),
                                   cache, w.scale)
    _, ref = oracle_decode(w)
    got = O.to_f32(from_dev(out).reshape(w.B, w.Hq, w.D), "bf16").astype(np.float64)
    assert output_error(got, ref, "bf16") <= TOL


def test_errors_are_status_codes(gpu):
    """Misuse returns a status code and leaves the cache unchanged."""
    from bsattn import BsattnError
    w = make_workload(3500, B=2, Hq=32, Hkv=8, T=64, Tb=64, dtype="f16", top_k=2, lens=[64, 0])
    cache = new_cache(w, mbps=4, num_pages=3)
    fill(cache, w, gpu)
    big = to_dev(np.zeros((1, 8, 300, 128), np.uint16), "f16", gpu)
    with pytest.raises(BsattnError) as e:
        cache.append(big, big)  # 364 tokens > max_blocks_per_seq * block_size = 256
    assert e.value.code == -4
    assert cache.offset == 64  # the failed call changed nothing
    small = big[:, :, :64].contiguous()
    with pytest.raises(BsattnError) as e:
        cache.append(small, small, seq_ids=[3])  # sequence id out of range
    assert e.value.code == -4
    mid = big[:, :, :192].contiguous()
    with pytest.raises(BsattnError) as e:
        cache.append(mid, mid, seq_ids=[1])  # needs 3 pages, 2 free
    assert e.value.code == -3
    assert cache.seqLen(1) == 0 and cache.freePages == 2


def test_graph_replay_matches_eager(gpu):
    """decode captured in a HIP graph: every replay, with eager work and
    synchronizations in between, equals the eager result."""
    import torch
    w = make_workload(3600, B=4, Hq=32, Hkv=8, T=3000, Tb=64, dtype="bf16", top_k=8)
    cache = new_cache(w)
    fill(cache, w, gpu)
    q = to_dev(w.q[:, :, None, :], "bf16", gpu)
    eager = cache.decode(q, w.scale)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        cache.decode(q, w.scale)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = cache.decode(q, w.scale)
    for r in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {r} differs"
        other = cache.decode(q, w.scale)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(other.view(torch.int16), eager.view(torch.int16))


def test_profiling_counts_launches(gpu):
    """bsattn_profile_*: eager launches are timed per kernel kind."""
    import torch
    from bsattn import _lib
    w = make_workload(3700, B=2, Hq=32, Hkv=8, T=4000, Tb=64, dtype="bf16", top_k=8)
    cache = new_cache(w)
    fill(cache, w, gpu)
    q = to_dev(w.q[:, :, None, :], "bf16", gpu)
    cache.profile(True)
    for _ in range(3):
        idx = cache.selectBlocks(q)
        cache.attend(q, idx, w.scale)
    cache.decode(q, w.scale)
    torch.cuda.synchronize()
    ms, n = cache.profileRead(_lib.KERNEL_ATTEND)
    assert n == 4 and ms > 0
    assert cache.profileRead(_lib.KERNEL_TOPK)[1] == 3
    # the decode is one fused launch (scoring and selection inside the
    # attention kernel): only the three selectBlocks calls launch k_score
    assert cache.profileRead(_lib.KERNEL_SCORE)[1] == 3
    assert cache.profileRead(_lib.KERNEL_COMBINE)[1] == 4
    cache.profile(False)
    assert cache.profileRead(_lib.KERNEL_ATTEND) == (0.0, 0)


@pytest.mark.parametrize("kv_bits", [0, 4])
def test_prompt_cache_round_trip(gpu, tmp_path, kv_bits):
    """savePromptCache / loadPromptCache (KVCache.swift:1244-1388) over real
    layer caches: the reloaded caches export the same state and summaries
    and decode bit-identically; the dense-compatible file loads into a
    cache through its KVCache / QuantizedKVCache entry."""
    import torch
    from bsattn import loadPromptCache, savePromptCache
    dt = "f16" if kv_bits else "bf16"
    layers = []
    for li in range(2):
        w = make_workload(3400 + li, B=2, Hq=32, Hkv=8, T=700, Tb=64, dtype=dt, top_k=4)
        c = new_cache(w, mbps=16, kv_bits=kv_bits)
        fill(c, w, gpu)
        layers.append((w, c))
    path = str(tmp_path / "prompt.safetensors")
    savePromptCache(path, [c for _, c in layers], {"model": "test"})

    def make(i, cls, ms, state):
        assert cls == "BlockSparseKVCache" and ms == layers[i][1].metaState
        return new_cache(layers[i][0], mbps=16, kv_bits=kv_bits)

    loaded, user = loadPromptCache(path, make)
    assert user == {"model": "test"}
    for (w, c), c2 in zip(layers, loaded):
        for a, b in zip(c.state, c2.state):
            assert torch.equal(a, b)
        for b in range(w.B):
            assert torch.equal(c.exportSummaries(b), c2.exportSummaries(b))
        q = to_dev(w.q[:, :, None, :], w.dtype, gpu)
        o1, o2 = c.decode(q, w.scale), c2.decode(q, w.scale)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2)
    # the dense-compatible file: reference class names, same arrays
    dpath = str(tmp_path / "dense.safetensors")
    savePromptCache(dpath, [c for _, c in layers], dense_compatible=True)
    want = "QuantizedKVCache" if kv_bits else "KVCache"
    loaded, _ = loadPromptCache(dpath, lambda i, cls, ms, st: (cls == want or pytest.fail(cls))
                                and new_cache(layers[i][0], mbps=16, kv_bits=kv_bits))
    for (w, c), c2 in zip(layers, loaded):
        for a, b in zip(c.state, c2.state):
            assert torch.equal(a, b)


def test_new_cache_per_layer_and_quantize_later(gpu):
    """newCache (LanguageModel.newCache's block-sparse form): one cache per
    layer with that layer's kv heads; attentionWithCacheUpdate steps every
    layer (each against the oracle), and maybeQuantizeKVCache with the same
    parameters converts the layers once quantizedKVStart is passed."""
    import torch
    import bsattn
    params = bsattn.GenerateParameters(kvBits=4, kvGroupSize=64, quantizedKVStart=200)
    layers = bsattn.newCache([8, 4], params, num_q_heads=32, max_seqs=2, max_tokens=1024,
                             dtype=torch.float16, top_k=2, device=0)
    assert [c.desc.num_kv_heads for c in layers] == [8, 4] and all(c.bits == 0 for c in layers)
    for li, cache in enumerate(layers):
        Hkv = cache.desc.num_kv_heads
        w = make_workload(3900 + li, B=2, Hq=32, Hkv=Hkv, T=300, Tb=64, dtype="f16", top_k=2,
                          lens=[300, 300])
        prompt = Workload(w.seed, 2, 32, Hkv, w.D, 64, "f16", [299, 299], 2, 1, 1)
        prompt.keys = [k[:, :299] for k in w.keys]
        prompt.values = [v[:, :299] for v in w.values]
        fill(cache, prompt, gpu)
        k = to_dev(np.stack([kk[:, 299:300] for kk in w.keys]), "f16", gpu)
        v = to_dev(np.stack([vv[:, 299:300] for vv in w.values]), "f16", gpu)
        q = to_dev(w.q[:, :, None, :], "f16", gpu)
        out = bsattn.attentionWithCacheUpdate(q, k, v, cache, w.scale)
        torch.cuda.synchronize()
        _, out_ref = oracle_decode(w)
        got = O.to_f32(from_dev(out).reshape(2, 32, w.D), "f16").astype(np.float64)
        assert output_error(got, out_ref, "f16") <= TOL
    bsattn.maybeQuantizeKVCache(layers, params.kvBits, params.kvGroupSize, params.quantizedKVStart)
    assert all(c.bits == 4 and c.seqLen(0) == 300 for c in layers)
