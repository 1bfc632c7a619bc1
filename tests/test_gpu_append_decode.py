"""bsattn_append_decode (the decode step of attentionWithCacheUpdate in one
call) against bsattn_append followed by bsattn_decode on a deep copy of the
same cache: outputs and selected blocks bit-identical at every step, across
block fills (the summary is written in the launch that also scores), new
pages, ragged lengths with interleaved pages, a reordered subset of the
sequences, GQA 4 / 8 / 16, the one-launch step over several splits per
(sequence, kv head), and the affine int4 cache (which takes the two calls);
after the last step also against the oracle."""
from __future__ import annotations

import numpy as np
import pytest

from common import (Workload, fill, from_dev, log, make_workload, new_cache, oracle_decode,
                    output_error, to_dev)
import oracle as O

pytestmark = pytest.mark.gpu

# dtype, Tb, Hq, Hkv, top_k, sink, recent, kv_bits, starting lengths, steps, seq_ids
CASES = {
    "bf16-tb64-g4": ("bf16", 64, 32, 8, 4, 1, 1, 0, [100, 190, 64, 255], 70, None),
    "f16-tb32-g8-subset": ("f16", 32, 32, 4, 3, 1, 2, 0, [31, 95, 200], 40, [2, 0]),
    "f16-tb32-g16-recent4": ("f16", 32, 64, 4, 3, 1, 4, 0, [40, 300, 129], 40, None),
    "int4": ("f16", 64, 32, 8, 2, 1, 1, 4, [100, 130], 30, None),
    # one launch over 3 splits per (sequence, kv head): the newest block's
    # slot (the last one) lies in split 2 while ranked and in split 1 while
    # every block is taken, and the blocks the tokens fill are folded in split 0
    "f16-tb32-splits-fill": ("f16", 32, 4, 2, 9, 1, 2, 0, [447, 60], 40, None),
    "bf16-tb64-splits-fill": ("bf16", 64, 8, 2, 9, 1, 2, 0, [830, 120], 80, None),
    # top_k 0 (sinks and recent only) over 2 splits, with block fills
    "f16-tb32-topk0": ("f16", 32, 8, 2, 0, 2, 3, 0, [300, 62], 40, None),
    # 2 sequences x 8 kv heads, 130 slots, more than 256 candidates: the
    # step's attention runs in 9-wave workgroups (15 splits, one workgroup
    # per CU), with block fills
    "bf16-tb64-g4-wide": ("bf16", 64, 32, 8, 128, 1, 1, 0, [20000, 19050], 40, None),
    "f16-tb32-g2-wide": ("f16", 32, 16, 8, 128, 1, 1, 0, [9990, 9650], 40, None),
}


@pytest.mark.parametrize("case", list(CASES))
def test_append_decode_equals_append_then_decode(gpu, case):
    log(f"[append-decode] {case}")
    run_case(gpu, case, 4100, *CASES[case])


def random_case(seed: int):
    r = np.random.default_rng(4300 + seed)
    bits = int(r.choice([0, 0, 4, 8]))
    dtype = "f16" if bits else str(r.choice(["f16", "bf16"]))
    Tb = int(r.choice([32, 64]))
    G = int(r.choice([1, 2, 4, 8, 16]))
    Hkv = int(r.choice([1, 2, 4]))
    B = int(r.integers(1, 5))
    # starting lengths near block boundaries, inside blocks and tiny
    lens0 = [int(r.choice([Tb - 1, Tb, 3 * Tb - 2, int(r.integers(1, 40 * Tb))])) for _ in range(B)]
    ids = None
    if B > 1 and seed % 3 == 0:
        ids = [int(x) for x in r.permutation(B)[: int(r.integers(1, B + 1))]]
    return (dtype, Tb, Hkv * G, Hkv, int(r.choice([1, 2, 3, 5, 9])), int(r.integers(0, 3)),
            int(r.choice([1, 2, 4])), bits, lens0, int(r.integers(10, 2 * Tb + 10)), ids)


@pytest.mark.parametrize("seed", range(16))
def test_append_decode_random(gpu, seed):
    """Seeded random shapes through the same checks: cache type (fp16, bf16,
    int4, int8), block size, GQA group, batch, starting lengths at and around
    block boundaries, top_k, sinks, recent blocks, steps (up to two block
    fills), and a reordered subset of the sequences."""
    c = random_case(seed)
    log(f"[append-decode random {seed}] {c}")
    run_case(gpu, f"random {seed}", 4400 + seed, *c)


def random_fused_case(seed: int):
    """16-bit caches with GQA groups of at most 4, where the step is one launch
    of the fused decode: batches of 1-6 sequences (one split per (sequence, kv
    head) at the larger ones, several at the smaller, where the newest
    block's slot can lie in any split), lengths at and around block
    boundaries."""
    r = np.random.default_rng(4700 + seed)
    Tb = int(r.choice([32, 64]))
    G = int(r.choice([1, 2, 4]))
    Hkv = int(r.choice([1, 2, 4, 8]))
    B = int(r.integers(1, 7))
    lens0 = [int(r.choice([Tb - 1, 2 * Tb - 3, int(r.integers(1, 9 * Tb)), int(r.integers(8 * Tb, 30 * Tb))]))
             for _ in range(B)]
    return (str(r.choice(["f16", "bf16"])), Tb, Hkv * G, Hkv, int(r.choice([0, 1, 4, 9, 20])),
            int(r.integers(0, 3)), int(r.choice([1, 2, 3])), 0, lens0, int(r.integers(Tb, 2 * Tb + 5)), None)


@pytest.mark.parametrize("seed", range(8))
def test_append_decode_random_fused(gpu, seed):
    c = random_fused_case(seed)
    log(f"[append-decode fused random {seed}] {c}")
    run_case(gpu, f"fused random {seed}", 4800 + seed, *c)


def one_launch_lengths(seed: int, n_ranked: int, n_short: int, m_ranked, m_short):
    """Starting lengths 64 m - d (d in [1, 60]): every sequence completes a
    block within the first 60 appended tokens; n_ranked with m in m_ranked
    (more candidates than top_k: the newest block takes the last slot), the
    rest in m_short (every block taken in order: the newest block's slot is
    nb - 1)."""
    r = np.random.default_rng(seed)
    ms = [int(r.integers(*m_ranked)) for _ in range(n_ranked)] + \
         [int(r.integers(*m_short)) for _ in range(n_short)]
    r.shuffle(ms)
    return [64 * m - int(r.integers(1, 61)) for m in ms]


# Shapes where bsattn_append_decode is one launch of the fused decode with
# several gather rounds per wave, the newest block past round 0:
#  - 32 sequences x 8 kv heads (256 pairs, as the decode loop of 32
#    sequences): one split, 8 waves, 5 rounds; ranked sequences put the newest
#    block in slot 33 = round 4 of wave 1, the short ones in slot nb - 1;
#  - 8 sequences x 8 kv heads, top_k 64 (66 slots): 4 splits, 8 waves, 3
#    rounds; the newest block's slot 65 is round 2 of wave 0 in split 1.
ONE_LAUNCH = {
    "b32-hkv8-k32-r5": ("f16", 64, 32, 8, 32, 1, 1, 0, one_launch_lengths(51, 24, 8, (36, 52), (4, 33)), 70, None),
    "b32-hkv8-k32-r5-bf16": ("bf16", 64, 32, 8, 32, 1, 1, 0, one_launch_lengths(52, 28, 4, (36, 45), (2, 30)), 66, None),
    "b8-hkv8-k64-s4-r3": ("f16", 64, 32, 8, 64, 1, 1, 0, one_launch_lengths(53, 6, 2, (68, 250), (10, 66)), 70, None),
}


@pytest.mark.parametrize("case", list(ONE_LAUNCH))
def test_append_decode_one_launch_rounds(gpu, case):
    """The one-launch step where the newest block is gathered in a round
    past the first (the decode loop of 32 sequences runs it so): bit-identical
    to append + decode at every step, one fused decode launch per step (plus
    the split combine with several splits; no append, scoring or selection
    launch), pages in a shuffled physical order, then selection, output and
    summaries against the oracle."""
    log(f"[append-decode one launch] {case}")
    run_case(gpu, case, 4900 + len(case), *ONE_LAUNCH[case], one_launch=True)


def run_case(gpu, case, wseed, dtype, Tb, Hq, Hkv, K, ns, nr, bits, lens0, steps, ids, one_launch=False):
    import torch
    from bsattn import _lib
    B = len(lens0)
    ids_l = list(range(B)) if ids is None else ids
    total = [l + (steps if b in ids_l else 0) for b, l in enumerate(lens0)]
    w = make_workload(wseed, B=B, Hq=Hq, Hkv=Hkv, T=max(total), Tb=Tb, dtype=dtype, top_k=K,
                      ns=ns, nr=nr, lens=total)
    a = new_cache(w, kv_bits=bits)
    w0 = Workload(w.seed, B, Hq, Hkv, w.D, Tb, dtype, lens0, K, ns, nr)
    w0.keys = [w.keys[b][:, :lens0[b]] for b in range(B)]
    w0.values = [w.values[b][:, :lens0[b]] for b in range(B)]
    if one_launch:
        a.shuffleFreePages(wseed)
        fill(a, w0, gpu)
    else:
        fill(a, w0, gpu, chunk=40)
    b_ = a.copy()
    if one_launch:
        a.profile(True)
    q = to_dev(w.q[ids_l][:, :, None, :], dtype, gpu)
    nsel = ns + nr + K
    cur = list(lens0)
    for s in range(steps):
        for b in ids_l:
            cur[b] += 1
        k = np.stack([w.keys[b][:, cur[b] - 1:cur[b]] for b in ids_l])
        v = np.stack([w.values[b][:, cur[b] - 1:cur[b]] for b in ids_l])
        kd, vd = to_dev(k, dtype, gpu), to_dev(v, dtype, gpu)
        ia = torch.empty((len(ids_l), Hkv, nsel), dtype=torch.int32, device=gpu)
        ib = torch.empty_like(ia)
        out_a = a.appendDecode(kd, vd, q, w.scale, seq_ids=ids, idx_out=ia)
        b_.append(kd, vd, seq_ids=ids)
        out_b = b_.decode(q, w.scale, seq_ids=ids, idx_out=ib)
        torch.cuda.synchronize()
        assert np.array_equal(ia.cpu().numpy(), ib.cpu().numpy()), f"step {s}: selected blocks differ"
        assert np.array_equal(from_dev(out_a), from_dev(out_b)), f"step {s}: outputs differ"
    if one_launch:
        # one fused decode launch per step (followed by the split combine
        # when a (sequence, kv head) has several splits), and no append,
        # scoring, summary or selection launch
        n_att = a.profileRead(_lib.KERNEL_ATTEND)[1]
        n_comb = a.profileRead(_lib.KERNEL_COMBINE)[1]
        others = {k: a.profileRead(getattr(_lib, k))[1] for k in
                  ("KERNEL_APPEND", "KERNEL_SCORE", "KERNEL_SUMMARY", "KERNEL_TOPK")}
        a.profile(False)
        assert n_att == steps and n_comb in (0, steps) and not any(others.values()), \
            f"not one decode launch per step: attend {n_att}, combine {n_comb}, others {others}"
    for b in range(B):
        assert a.seqLen(b) == b_.seqLen(b) == cur[b]
    if bits == 0:
        for b in ids_l:
            assert np.array_equal(from_dev(a.exportSummaries(b)), from_dev(b_.exportSummaries(b)))
        wl = Workload(w.seed, len(ids_l), Hq, Hkv, w.D, Tb, dtype, [cur[b] for b in ids_l], K, ns, nr)
        wl.q = w.q[ids_l]
        wl.keys = [w.keys[b][:, :cur[b]] for b in ids_l]
        wl.values = [w.values[b][:, :cur[b]] for b in ids_l]
        idx_ref, out_ref = oracle_decode(wl)
        assert np.array_equal(ia.cpu().numpy(), idx_ref), "selected blocks differ from the oracle"
        got = O.to_f32(from_dev(out_a).reshape(len(ids_l), Hq, w.D), dtype).astype(np.float64)
        err = output_error(got, out_ref, dtype)
        assert err <= 2e-3, f"output error {err:.3g}"
        log(f"[append-decode] {case} err={err:.3g}")


def test_append_decode_errors(gpu):
    """Shape / range errors are reported, and nothing is appended."""
    import torch
    w = make_workload(4200, B=2, Hq=32, Hkv=8, T=130, Tb=64, dtype="f16", top_k=1, lens=[130, 130])
    c = new_cache(w, mbps=3)
    fill(c, w, gpu)
    k = torch.zeros((2, 8, 1, 128), dtype=torch.float16, device=gpu)
    q = torch.zeros((2, 32, 1, 128), dtype=torch.float16, device=gpu)
    with pytest.raises(ValueError):
        c.appendDecode(k[:1], k[:1], q, 0.1)
    c.appendDecode(k, k, q, 0.1)   # 131 tokens: the third block
    with pytest.raises(Exception):
        for _ in range(64):        # the 193rd token needs a fourth block
            c.appendDecode(k, k, q, 0.1)
    assert c.seqLen(0) == 192 and c.seqLen(1) == 192
