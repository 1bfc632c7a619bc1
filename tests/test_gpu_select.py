"""Block-wide selection (candidate sets larger than one wave's selection, or
top_k above it) and MFMA scoring for wide GQA groups with the exact
rescoring band: selected indices bit-exact against the oracle, outputs within
2e-3 (net of the output rounding)."""
from __future__ import annotations

import numpy as np
import pytest

from common import fill, from_dev, log, make_workload, new_cache, oracle_decode, output_error, to_dev
import oracle as O

pytestmark = pytest.mark.gpu

TOL = 2e-3


def check(cache, w, gpu, decode=True):
    import torch
    q = to_dev(w.q[:, :, None, :], w.dtype, gpu)
    idx_ref, out_ref = oracle_decode(w)
    idx = cache.selectBlocks(q)
    out = cache.attend(q, idx, w.scale)
    torch.cuda.synchronize()
    got = idx.cpu().numpy()
    bad = np.argwhere(got != idx_ref)
    assert bad.size == 0, f"selected blocks differ at {bad[:5]}: {got[tuple(bad[0][:2])][:12]} vs {idx_ref[tuple(bad[0][:2])][:12]}"
    a = from_dev(out).reshape(w.B, w.Hq, w.D)
    err = output_error(O.to_f32(a, w.dtype).astype(np.float64), out_ref, w.dtype)
    assert err <= TOL, f"output error {err:.3g}"
    if decode:
        out2 = cache.decode(q, w.scale)
        torch.cuda.synchronize()
        assert np.array_equal(from_dev(out2).reshape(w.B, w.Hq, w.D), a), "decode != select + attend"
    return err


@pytest.mark.parametrize("dtype,Hq,Hkv,Tb,K", [
    ("bf16", 16, 4, 64, 32), ("f16", 16, 4, 32, 5), ("bf16", 4, 4, 32, 300), ("f16", 4, 2, 64, 64),
])
def test_block_select_exact_scores(gpu, dtype, Hq, Hkv, Tb, K):
    """G <= 4: canonical VALU scores, k_select over 1000 - 5000 candidates
    (ragged, including sequences below and above one wave's limit)."""
    lens = [Tb * 5000 - 7, Tb * 1100, Tb * 700 + 3, Tb * 30, Tb * 2500 + 1] if Tb == 32 else \
        [Tb * 2600 - 7, Tb * 1100, Tb * 700 + 3, Tb * 30]
    log(f"[select] {dtype} G={Hq // Hkv} Tb={Tb} K={K}")
    w = make_workload(5000 + Hq + Tb + K, B=len(lens), Hq=Hq, Hkv=Hkv, T=max(lens), Tb=Tb, dtype=dtype,
                      top_k=K, ns=2, nr=3, lens=lens, salient_frac=0.01)
    cache = new_cache(w)
    fill(cache, w, gpu)
    err = check(cache, w, gpu)
    log(f"[select] err={err:.3g}")


@pytest.mark.parametrize("dtype,Hq,Hkv,Tb,K", [
    ("bf16", 64, 4, 32, 128), ("f16", 64, 4, 32, 128), ("bf16", 32, 4, 64, 40), ("f16", 16, 2, 64, 7),
])
def test_wide_group_mfma_band(gpu, dtype, Hq, Hkv, Tb, K):
    """G = 8 / 16 with more than one wave's candidates: MFMA scores, exact
    rescoring of the band, bit-exact selection."""
    lens = [Tb * 3000 + 5, Tb * 1030, Tb * 200, Tb * 4096] if Tb == 32 else \
        [Tb * 2000 + 5, Tb * 1030, Tb * 200, Tb * 2500]
    log(f"[band] {dtype} G={Hq // Hkv} Tb={Tb} K={K}")
    w = make_workload(5100 + Hq + Tb + K, B=len(lens), Hq=Hq, Hkv=Hkv, T=max(lens), Tb=Tb, dtype=dtype,
                      top_k=K, ns=1, nr=4, lens=lens, salient_frac=0.01)
    cache = new_cache(w)
    fill(cache, w, gpu)
    err = check(cache, w, gpu)
    log(f"[band] err={err:.3g}")


@pytest.mark.parametrize("dtype,Hq,Hkv", [("f16", 64, 4), ("bf16", 32, 4)])
def test_wide_group_partial_last_chunk(gpu, dtype, Hq, Hkv):
    """The scoring chunks' floors at each kind of last chunk (256 candidates a
    chunk, 16 per tile; the longest sequence's 4091 candidates make 16 chunks
    and a floor rank of 128 / 16 = 8): 3880 candidates leave 40 in the last
    chunk (3 tiles: the floor is that chunk's 8th largest score), 3184 leave
    112 (7 tiles, likewise), 2673 leave 113 (8 tiles, the last holding one
    candidate: the 8th largest tile maximum), 4091 leave 251."""
    Tb = 32
    lens = [3884 * Tb + 22, 3188 * Tb + 1, 2678 * Tb, 4096 * Tb]
    log(f"[last chunk] {dtype} G={Hq // Hkv}")
    w = make_workload(5300 + Hq, B=len(lens), Hq=Hq, Hkv=Hkv, T=max(lens), Tb=Tb, dtype=dtype,
                      top_k=128, ns=1, nr=4, lens=lens, salient_frac=0.01)
    cache = new_cache(w)
    fill(cache, w, gpu)
    err = check(cache, w, gpu)
    log(f"[last chunk] err={err:.3g}")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_wide_group_ties_and_duplicates(gpu, dtype):
    """Sequence 0: every block has the same keys (all scores tie: the band is
    every candidate, lowest indices win).  Sequence 1: a few blocks copied
    many times near the top (exact ties inside the band)."""
    Tb = 32
    lens = [Tb * 1500, Tb * 1600 + 11]
    w = make_workload(5200, B=2, Hq=64, Hkv=4, T=max(lens), Tb=Tb, dtype=dtype, top_k=50, ns=1, nr=4,
                      lens=lens, salient_frac=0.01)
    for h in range(w.Hkv):
        blk = w.keys[0][h][:Tb].copy()
        for j in range(lens[0] // Tb):
            w.keys[0][h][j * Tb:(j + 1) * Tb] = blk
        rng = np.random.default_rng(h)
        for src in rng.choice(lens[1] // Tb - 10, 5, replace=False) + 5:
            for dst in rng.choice(lens[1] // Tb - 10, 20, replace=False) + 5:
                w.keys[1][h][dst * Tb:(dst + 1) * Tb] = w.keys[1][h][src * Tb:(src + 1) * Tb]
    cache = new_cache(w)
    fill(cache, w, gpu)
    check(cache, w, gpu)
    q = to_dev(w.q[:, :, None, :], w.dtype, gpu)
    idx = cache.selectBlocks(q).cpu().numpy()
    nb = lens[0] // Tb
    assert list(idx[0, 0][:52]) == list(range(51)) + [nb - 4]


@pytest.mark.parametrize("T_blocks,Hq,Hkv,K", [(300, 32, 8, 20), (2500, 32, 8, 40), (1500, 64, 4, 30)])
def test_nonfinite_scores_select_like_oracle(gpu, T_blocks, Hq, Hkv, K):
    """Keys holding +-inf give infinite or NaN block scores (NaN sorts lowest,
    -0 == +0); selection stays bit-exact on the one-wave, workgroup and
    MFMA-band paths.  Indices only: the attention of such keys is NaN."""
    import torch
    Tb = 64
    w = make_workload(5300 + T_blocks + Hq, B=2, Hq=Hq, Hkv=Hkv, T=T_blocks * Tb, Tb=Tb, dtype="f16",
                      top_k=K, ns=1, nr=2)
    rng = np.random.default_rng(T_blocks)
    for b in range(w.B):
        for h in range(w.Hkv):
            for j in rng.choice(T_blocks - 4, 6, replace=False) + 1:
                w.keys[b][h][j * Tb + 3, rng.integers(0, 128)] = 0x7C00        # +inf
            for j in rng.choice(T_blocks - 4, 4, replace=False) + 1:
                w.keys[b][h][j * Tb + 5, rng.integers(0, 128)] = 0xFC00        # -inf
            j = int(rng.integers(1, T_blocks - 4))
            w.keys[b][h][j * Tb + 1, 7] = 0x7C00                                # +inf and -inf: NaN
            w.keys[b][h][j * Tb + 2, 7] = 0xFC00
    cache = new_cache(w)
    fill(cache, w, gpu)
    q = to_dev(w.q[:, :, None, :], w.dtype, gpu)
    idx_ref, _ = oracle_decode(w)
    idx = cache.selectBlocks(q)
    idx2 = torch.empty_like(idx)
    cache.decode(q, w.scale, idx_out=idx2)
    torch.cuda.synchronize()
    got = idx.cpu().numpy()
    assert np.array_equal(got, idx_ref), f"differ at {np.argwhere(got != idx_ref)[:5]}"
    assert np.array_equal(idx2.cpu().numpy(), idx_ref)


@pytest.mark.parametrize("dtype,Hq,Hkv,Tb,K,lo,hi,mult", [
    ("f16", 64, 4, 32, 128, 500, 700, 4.0),     # the top blocks in three scoring chunks
    ("bf16", 64, 4, 32, 128, 1000, 1128, 3.0),  # exactly K boosted blocks, side by side
    ("f16", 32, 4, 64, 40, 10, 2000, 1.02),     # most blocks slightly boosted: the floor is low
])
def test_wide_group_clustered_top_blocks(gpu, dtype, Hq, Hkv, Tb, K, lo, hi, mult):
    """Wide groups whose best blocks sit side by side: the wave floors of the
    MFMA scoring then come from waves without any of them, and the candidates
    kept for the compacted selection (or its fallback to all of them) must
    still give the canonical selection."""
    lens = [Tb * 3000 + 7, Tb * 2600]
    w = make_workload(5600 + lo + K, B=len(lens), Hq=Hq, Hkv=Hkv, T=max(lens), Tb=Tb, dtype=dtype,
                      top_k=K, ns=1, nr=4, lens=lens)
    for b in range(w.B):
        for h in range(w.Hkv):
            k = O.to_f32(w.keys[b][h], dtype)
            k[lo * Tb:hi * Tb] *= mult
            w.keys[b][h][:] = O.from_f32(k.astype(np.float32), dtype)
    cache = new_cache(w)
    fill(cache, w, gpu)
    err = check(cache, w, gpu)
    log(f"[clustered] {dtype} G={Hq // Hkv} [{lo}, {hi}) x{mult} err={err:.3g}")


@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (64, 4)])
def test_fused_dot_steps_select_like_oracle(gpu, Hq, Hkv):
    """bf16 scores whose in-chunk steps differ fused and unfused: in block 50
    of kv head 0, chunk 0 folds (-2^127)(1), then 2^64 * 2^64 = 2^128 (out of
    fp32's range alone), then (-2^127)(1).  Fused, each step rounds a*b + acc
    once and the chunk sums to 0, so the block scores like any other; with a
    separate multiply the second product would be +inf and the block the
    top one.  Every other block is zero in dims 0 - 2.  The VALU scoring
    (G = 4) and the MFMA path (G = 16, whose bound is then not finite, so
    every candidate is rescored) must select like the oracle.  Indices
    only: the attention of such keys overflows."""
    import torch
    Tb, K, nblk = 64, 20, 300
    w = make_workload(5800 + Hq, B=1, Hq=Hq, Hkv=Hkv, T=nblk * Tb, Tb=Tb, dtype="bf16", top_k=K, ns=1, nr=1)
    k = O.to_f32(w.keys[0][0], "bf16")
    k[:, :3] = 0.0
    k[50 * Tb:51 * Tb, :3] = [1.0, 2.0 ** 64, 1.0]
    w.keys[0][0][:] = O.from_f32(k, "bf16")
    q = O.to_f32(w.q[0, :w.G], "bf16")
    q[:, :3] = [-(2.0 ** 127), 2.0 ** 64, -(2.0 ** 127)]
    w.q[0, :w.G] = O.from_f32(q, "bf16")
    summ = O.summaries(w.keys[0][0], Tb, "bf16")
    sc = O.score_blocks(w.q[0, :w.G], summ, "bf16")
    assert np.isfinite(sc[50]) and sc[50] < np.sort(sc[1:nblk - 1])[-K]  # not selected when fused
    cache = new_cache(w)
    fill(cache, w, gpu)
    qd = to_dev(w.q[:, :, None, :], w.dtype, gpu)
    idx_ref, _ = oracle_decode(w)
    assert 50 not in idx_ref[0, 0]
    got = cache.selectBlocks(qd).cpu().numpy()
    idx2 = torch.empty_like(torch.from_numpy(got)).to(gpu)
    cache.decode(qd, w.scale, idx_out=idx2)
    torch.cuda.synchronize()
    assert np.array_equal(got, idx_ref), f"differ at {np.argwhere(got != idx_ref)[:5]}"
    assert np.array_equal(idx2.cpu().numpy(), idx_ref)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("case", ["gap", "ties"])
def test_wide_group_band_at_kth(gpu, dtype, case):
    """G = 16 over 2095 - 2996 candidates (MFMA scores, certified floor):
    the band of bins around the K-th approximate score.
    gap: K blocks whose keys are 0.5 .. 0.89 times the group's first query
    row score far above the rest, so the band holds only places still to
    fill and nothing is rescored.
    ties: twelve blocks hold the keys of the block ranked K - 4, so the K-th
    exact score falls among equal ones: the band is rescored and its ties go
    to the lower block indices."""
    Tb, K = 32, 40
    lens = [Tb * 3000 + 5, Tb * 2100]
    w = make_workload(5700 + len(case) + len(dtype), B=len(lens), Hq=64, Hkv=4, T=max(lens), Tb=Tb,
                      dtype=dtype, top_k=K, ns=1, nr=4, lens=lens)
    rng = np.random.default_rng(len(case) + len(dtype))
    for b in range(w.B):
        nb = (lens[b] + Tb - 1) // Tb
        cand = np.arange(w.ns, nb - w.nr)
        for h in range(w.Hkv):
            if case == "gap":
                q0 = O.to_f32(w.q[b, h * w.G], dtype).astype(np.float64)
                for i, j in enumerate(rng.choice(cand, K, replace=False)):
                    row = ((0.5 + 0.01 * i) * q0).astype(np.float32)
                    w.keys[b][h][j * Tb:(j + 1) * Tb] = O.from_f32(np.tile(row, (Tb, 1)), dtype)
            else:
                summ = O.summaries(w.keys[b][h][:(nb - 1) * Tb], Tb, dtype)
                sc = O.score_blocks(w.q[b, h * w.G:(h + 1) * w.G], summ, dtype)
                src = cand[np.argsort(-sc[cand], kind="stable")][K - 5]
                for j in rng.choice(np.setdiff1d(cand, [src]), 11, replace=False):
                    w.keys[b][h][j * Tb:(j + 1) * Tb] = w.keys[b][h][src * Tb:(src + 1) * Tb]
    cache = new_cache(w)
    fill(cache, w, gpu)
    err = check(cache, w, gpu)
    log(f"[band at K-th] {case} {dtype} err={err:.3g}")


@pytest.mark.parametrize("dtype,Hq,Hkv,Tb,K,scale", [
    ("f16", 64, 4, 32, 128, 1e-3), ("bf16", 32, 4, 64, 40, 1e-2), ("f16", 16, 4, 64, 32, 1e-3),
])
def test_near_equal_scores(gpu, dtype, Hq, Hkv, Tb, K, scale):
    """Every block's keys are one shared row plus small noise, so the scores
    crowd within a few bound widths: the compacted-list selection must fall
    back to the full workgroup path (wide groups) or stay exact (G = 4)."""
    lens = [Tb * 3000 + 9, Tb * 1500]
    w = make_workload(5400 + Hq + K, B=len(lens), Hq=Hq, Hkv=Hkv, T=max(lens), Tb=Tb, dtype=dtype,
                      top_k=K, ns=1, nr=2, lens=lens)
    rng = np.random.default_rng(K)
    for b in range(w.B):
        for h in range(w.Hkv):
            base = rng.standard_normal(128)
            noise = rng.standard_normal((w.keys[b][h].shape[0], 128)) * scale
            w.keys[b][h][:] = O.from_f32((base[None, :] + noise).astype(np.float32), w.dtype)
    cache = new_cache(w)
    fill(cache, w, gpu)
    err = check(cache, w, gpu)
    log(f"[near-equal] {dtype} G={Hq // Hkv} err={err:.3g}")


@pytest.mark.parametrize("case", ["plain", "ties", "near"])
def test_decode_workgroup_selection(gpu, case):
    """Decode with 1029 - 2048 candidate blocks: the selection runs inside the
    attention workgroup with every wave holding a share of the candidates.
    Indices (written by the decode itself) bit-exact against the oracle for
    ordinary, all-tied / duplicated and near-equal scores; outputs within
    the tolerance."""
    import torch
    Tb = 64
    lens = [Tb * 2050, Tb * 1030 + 5, Tb * 1800 - 3]      # 2048, 1029, 1797 candidates
    w = make_workload(5500 + len(case), B=len(lens), Hq=8, Hkv=2, T=max(lens), Tb=Tb, dtype="bf16",
                      top_k=40, ns=1, nr=1, lens=lens, salient_frac=0.01 if case == "plain" else 0.0)
    rng = np.random.default_rng(len(case))
    for h in range(w.Hkv):
        if case == "ties":
            blk = w.keys[0][h][:Tb].copy()
            for j in range(lens[0] // Tb):
                w.keys[0][h][j * Tb:(j + 1) * Tb] = blk
            for b in (1, 2):
                nbf = lens[b] // Tb
                for src in rng.choice(nbf - 10, 6, replace=False) + 5:
                    for dst in rng.choice(nbf - 10, 25, replace=False) + 5:
                        w.keys[b][h][dst * Tb:(dst + 1) * Tb] = w.keys[b][h][src * Tb:(src + 1) * Tb]
        elif case == "near":
            for b in range(w.B):
                base = rng.standard_normal(128)
                noise = rng.standard_normal((w.keys[b][h].shape[0], 128)) * 1e-3
                w.keys[b][h][:] = O.from_f32((base[None, :] + noise).astype(np.float32), w.dtype)
    cache = new_cache(w)
    fill(cache, w, gpu)
    q = to_dev(w.q[:, :, None, :], w.dtype, gpu)
    idx_ref, out_ref = oracle_decode(w)
    idx = torch.full((w.B, w.Hkv, idx_ref.shape[2]), -7, dtype=torch.int32, device=gpu)
    out = cache.decode(q, w.scale, idx_out=idx)
    torch.cuda.synchronize()
    got = idx.cpu().numpy()
    bad = np.argwhere(got != idx_ref)
    assert bad.size == 0, f"selected blocks differ at {bad[:5]}"
    a = from_dev(out).reshape(w.B, w.Hq, w.D)
    err = output_error(O.to_f32(a, w.dtype).astype(np.float64), out_ref, w.dtype)
    assert err <= TOL, f"output error {err:.3g}"
    if case == "ties":
        assert list(got[0, 0][:41]) == list(range(41))
    log(f"[wg-select] {case} err={err:.3g}")


# (B, Hq, Hkv, K, lengths in blocks): a 4-wave shape and a 9-wave one
# (2 sequences x 8 kv heads x 130 slots = 240 workgroups of 9 waves)
ALL_KEYS_SHAPES = {
    "w4": (32, 8, 2, 40, [514, 300, 70, 40]),
    "w9": (64, 32, 8, 128, [514, 331]),
}


@pytest.mark.parametrize("shape", list(ALL_KEYS_SHAPES))
@pytest.mark.parametrize("case", ["plain", "ties", "near", "crowd"])
def test_decode_all_keys_selection(gpu, case, shape):
    """Decode with at most 512 candidate blocks: every wave of the attention
    workgroup holds all candidates and selects with one workgroup barrier.
    Sequences of 512, 329, 67 (and 38, fewer than top_k: every block)
    candidates; ordinary scores, all-tied and duplicated blocks, near-equal
    scores, and a crowd of near-equal scores under a few large ones (the
    K-th key's value bin then holds more than 64 keys, so a second pass bins
    by key bits).  Indices (written by the decode itself) bit-exact against
    the oracle, outputs within the tolerance, decode == select + attend."""
    import torch
    Tb = 64
    B, Hq, Hkv, K, nblk = ALL_KEYS_SHAPES[shape]
    lens = [Tb * n - (3 if i % 2 else 0) for i, n in enumerate(nblk)][:B]
    w = make_workload(5600 + len(case) + Hkv, B=len(lens), Hq=Hq, Hkv=Hkv, T=max(lens), Tb=Tb, dtype="bf16",
                      top_k=K, ns=1, nr=1, lens=lens, salient_frac=0.01 if case == "plain" else 0.0)
    rng = np.random.default_rng(len(case) + Hkv)
    for b in range(w.B):
        nbf = lens[b] // Tb
        for h in range(w.Hkv):
            if case == "ties":
                if b == 0:
                    blk = w.keys[b][h][:Tb].copy()
                    for j in range(nbf):
                        w.keys[b][h][j * Tb:(j + 1) * Tb] = blk
                elif nbf > 20:
                    for src in rng.choice(nbf - 10, 4, replace=False) + 5:
                        for dst in rng.choice(nbf - 10, min(25, nbf - 10), replace=False) + 5:
                            w.keys[b][h][dst * Tb:(dst + 1) * Tb] = w.keys[b][h][src * Tb:(src + 1) * Tb]
            elif case in ("near", "crowd"):
                base = rng.standard_normal(128)
                noise = rng.standard_normal((w.keys[b][h].shape[0], 128)) * (1e-3 if case == "near" else 2e-4)
                rows = base[None, :] + noise
                if case == "crowd" and nbf > 12:
                    for j in rng.choice(nbf - 4, 3, replace=False) + 1:
                        rows[j * Tb:(j + 1) * Tb] *= 6.0
                w.keys[b][h][:] = O.from_f32(rows.astype(np.float32), w.dtype)
    cache = new_cache(w)
    fill(cache, w, gpu)
    q = to_dev(w.q[:, :, None, :], w.dtype, gpu)
    idx_ref, out_ref = oracle_decode(w)
    idx = torch.full((w.B, w.Hkv, idx_ref.shape[2]), -7, dtype=torch.int32, device=gpu)
    out = cache.decode(q, w.scale, idx_out=idx)
    sel = cache.selectBlocks(q)
    out2 = cache.attend(q, sel, w.scale)
    torch.cuda.synchronize()
    got = idx.cpu().numpy()
    bad = np.argwhere(got != idx_ref)
    assert bad.size == 0, f"selected blocks differ at {bad[:5]}"
    assert np.array_equal(sel.cpu().numpy(), idx_ref)
    a = from_dev(out).reshape(w.B, w.Hq, w.D)
    assert np.array_equal(a, from_dev(out2).reshape(w.B, w.Hq, w.D)), "decode != select + attend"
    err = output_error(O.to_f32(a, w.dtype).astype(np.float64), out_ref, w.dtype)
    assert err <= TOL, f"output error {err:.3g}"
    if case == "ties":
        assert list(got[0, 0][:K + 1]) == list(range(K + 1))
    log(f"[all-keys select] {case} {shape} err={err:.3g}")
