"""Multi-token decode (speculative verify, Evaluate.swift:862-870): L query
tokens per sequence after their L keys / values were appended; query i sees
the first T - L + 1 + i tokens and selects its own blocks there.  Checked
bit for bit against L single-token decodes run one after another (append a
token, decode it), and each query against the oracle on its prefix."""
from __future__ import annotations

import numpy as np
import pytest

from common import fill, from_dev, log, make_workload, new_cache, output_error, to_dev
import oracle as O

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _split(w, L):
    """(prefix keys / values per sequence, the L new tokens' keys / values)"""
    pre_k = [np.ascontiguousarray(k[:, :-L]) for k in w.keys]
    pre_v = [np.ascontiguousarray(v[:, :-L]) for v in w.values]
    new_k = np.stack([k[:, -L:] for k in w.keys])
    new_v = np.stack([v[:, -L:] for v in w.values])
    return pre_k, pre_v, new_k, new_v


def _queries(w, L, seed):
    # L query tokens per sequence: [B, Hq, L, D]
    return O.fill_normal(seed, 0, 0, (w.B, w.Hq, L, w.D), w.dtype)


def _prefix_cache(w, gpu, pre_k, pre_v, kv_bits):
    c = new_cache(w, kv_bits=kv_bits)
    for b in range(w.B):
        c.append(to_dev(pre_k[b][None], w.dtype, gpu), to_dev(pre_v[b][None], w.dtype, gpu), seq_ids=[b])
    return c


@pytest.mark.parametrize("dtype,Hq,Hkv,Tb,K,L,kv_bits,lens", [
    ("bf16", 32, 8, 64, 8, 4, 0, [4000, 2501]),           # fused selection, G = 4, 4 heads x 4 tokens
    ("f16", 32, 8, 64, 16, 5, 4, [6000, 3333]),           # int4 cache
    ("f16", 64, 4, 32, 40, 3, 0, [40000, 33000]),         # > 1024 candidates: MFMA band + workgroup select
    ("bf16", 16, 2, 64, 4, 8, 0, [64 * 7 + 3, 64 * 9]),   # a verify pass crossing block boundaries
])
def test_multi_decode_equals_sequential_decodes(gpu, dtype, Hq, Hkv, Tb, K, L, kv_bits, lens):
    import torch
    log(f"[multi] {dtype} G={Hq // Hkv} Tb={Tb} K={K} L={L} bits={kv_bits}")
    w = make_workload(6000 + Hq + L + kv_bits, B=len(lens), Hq=Hq, Hkv=Hkv, T=max(lens), Tb=Tb,
                      dtype=dtype, top_k=K, ns=1, nr=2, lens=lens, salient_frac=0.01)
    pre_k, pre_v, new_k, new_v = _split(w, L)
    qm = _queries(w, L, 6100 + L)
    # one pass: append L, decode L queries
    a = _prefix_cache(w, gpu, pre_k, pre_v, kv_bits)
    a.append(to_dev(new_k, dtype, gpu), to_dev(new_v, dtype, gpu))
    qd = to_dev(qm, dtype, gpu)
    idx_m = torch.empty((w.B, L, Hkv, a.nselMax), dtype=torch.int32, device=gpu)
    out_m = a.decodeMulti(qd, w.scale, idx_out=idx_m)
    # L passes: append a token, decode it
    s = _prefix_cache(w, gpu, pre_k, pre_v, kv_bits)
    for i in range(L):
        s.append(to_dev(np.ascontiguousarray(new_k[:, :, i:i + 1]), dtype, gpu),
                 to_dev(np.ascontiguousarray(new_v[:, :, i:i + 1]), dtype, gpu))
        qi = to_dev(np.ascontiguousarray(qm[:, :, i:i + 1]), dtype, gpu)
        idx_i = torch.empty((w.B, Hkv, s.nselMax), dtype=torch.int32, device=gpu)
        out_i = s.decode(qi, w.scale, idx_out=idx_i)
        torch.cuda.synchronize()
        assert torch.equal(idx_m[:, i], idx_i), f"query {i}: selections differ"
        assert np.array_equal(from_dev(out_m[:, :, i:i + 1]), from_dev(out_i)), f"query {i}: outputs differ"
    # every query against the oracle on its prefix (16-bit caches)
    if kv_bits == 0:
        got = from_dev(out_m)
        for i in range(L):
            for b in range(w.B):
                T_i = lens[b] - L + 1 + i
                idx_b = idx_m[b, i].cpu().numpy()
                for h in range(Hkv):
                    ri, _, ro = O.decode_head(qm[b, h * w.G:(h + 1) * w.G, i], w.keys[b][h][:T_i],
                                              w.values[b][h][:T_i], Tb, w.ns, w.nr, K, w.scale, dtype)
                    assert np.array_equal(idx_b[h], ri), f"seq {b} query {i} head {h}: selection"
                    err = output_error(O.to_f32(got[b, h * w.G:(h + 1) * w.G, i], dtype).astype(np.float64),
                                       ro, dtype)
                    assert err <= TOL, f"seq {b} query {i} head {h}: error {err:.3g}"


def _random_multi(seed: int):
    r = np.random.default_rng(6500 + seed)
    kv_bits = int(r.choice([0, 0, 4, 8]))
    dtype = "f16" if kv_bits else str(r.choice(["f16", "bf16"]))
    Tb = int(r.choice([32, 64]))
    G = int(r.choice([1, 2, 4, 8, 16]))
    Hkv = int(r.choice([1, 2, 4]))
    L = int(r.integers(2, 13))
    lens = [int(r.integers(L + 1, int(r.choice([40, 900])) * Tb)) for _ in range(int(r.integers(1, 4)))]
    return dtype, Hkv * G, Hkv, Tb, int(r.choice([2, 5, 16, 33, 70])), L, kv_bits, lens


@pytest.mark.parametrize("seed", range(12))
def test_multi_decode_random(gpu, seed):
    """Seeded random shapes through the same checks: cache type, block size,
    GQA group, top_k, 2 - 12 query tokens, ragged lengths up to 900 blocks."""
    c = _random_multi(seed)
    log(f"[multi random {seed}] {c}")
    test_multi_decode_equals_sequential_decodes(gpu, *c)


def test_attention_with_cache_update_verify_pass(gpu):
    """attentionWithCacheUpdate with L > 1 and the causal mask appends the
    L tokens and runs the multi-token decode; other masks are refused."""
    import torch
    from bsattn import attentionWithCacheUpdate
    w = make_workload(6200, B=2, Hq=32, Hkv=8, T=3000, Tb=64, dtype="bf16", top_k=8)
    L = 3
    pre_k, pre_v, nk, nv = _split(w, L)
    new_k, new_v = to_dev(nk, "bf16", gpu), to_dev(nv, "bf16", gpu)
    qm = to_dev(_queries(w, L, 6201), "bf16", gpu)
    a = _prefix_cache(w, gpu, pre_k, pre_v, 0)
    b = _prefix_cache(w, gpu, pre_k, pre_v, 0)
    with pytest.raises(ValueError):
        attentionWithCacheUpdate(qm, new_k, new_v, a, w.scale, mask="none")
    assert a.offset == 3000 - L  # refused before the update
    o1 = attentionWithCacheUpdate(qm, new_k, new_v, a, w.scale, mask=a.makeMask(L))
    b.append(new_k, new_v)
    o2 = b.decodeMulti(qm, w.scale)
    torch.cuda.synchronize()
    assert a.offset == 3000 and torch.equal(o1, o2)


def test_multi_decode_argument_errors(gpu):
    import torch
    from bsattn import BsattnError
    w = make_workload(6300, B=1, Hq=32, Hkv=8, T=100, Tb=64, dtype="bf16", top_k=2)
    c = new_cache(w)
    fill(c, w, gpu)
    q17 = torch.zeros((1, 32, 17, 128), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(BsattnError):
        c.decodeMulti(q17, 1.0)  # more than 16 queries
    c2 = new_cache(w)
    c2.append(to_dev(np.ascontiguousarray(w.keys[0][None, :, :2]), "bf16", gpu),
              to_dev(np.ascontiguousarray(w.values[0][None, :, :2]), "bf16", gpu))
    q3 = torch.zeros((1, 32, 3, 128), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(BsattnError):
        c2.decodeMulti(q3, 1.0)  # 2 tokens, 3 queries


def _oracle_query(qh, keys, values, T, Tb, ns, nr, K, scale, dtype, bits):
    """oracle selection and output of one kv head's group of queries qh
    [G, D] over the first T tokens of keys / values [T_all, D] (16-bit, or
    quantized on append by the affine codec when bits)."""
    if bits == 0:
        idx, _, out = O.decode_head(qh, keys[:T], values[:T], Tb, ns, nr, K, scale, dtype)
        return idx, out
    kq = O.quantize(np.ascontiguousarray(keys[:T]), bits, 64)
    vq = O.quantize(np.ascontiguousarray(values[:T]), bits, 64)
    summ = O.summaries_q(*kq, Tb, bits, 64)
    idx, n = O.select(O.score_blocks(qh, summ, "f16"), T, Tb, ns, nr, K)
    return idx, O.attend_q(qh, kq, vq, Tb, bits, 64, idx[:n], scale)


@pytest.mark.parametrize("dtype,Tb,kv_bits", [("bf16", 64, 0), ("f16", 32, 0), ("f16", 64, 4),
                                               ("f16", 32, 4)])
def test_trim_rewinds_a_completed_block(gpu, dtype, Tb, kv_bits):
    """A speculative round that is mostly rejected (Evaluate.swift:909-911 ->
    trimPromptCache, KVCache.swift:1520-1524, 396-402): 5 draft tokens
    complete a block (its summary is written) and start the next; trimming 4
    of them makes the completed block partial again; 3 different tokens then
    refill it, so its summary must be recomputed from the new token.  After
    each pass the summaries are bit-exact and every query of decodeMulti
    matches the oracle on its own prefix of the accepted sequence."""
    import torch
    L1, REJ, L2 = 5, 4, 3
    T0 = [7 * Tb - 2, 9 * Tb - 1]
    log(f"[trim-rewind] {dtype} Tb={Tb} bits={kv_bits}")
    w = make_workload(6400 + Tb + kv_bits, B=2, Hq=32, Hkv=8, T=max(T0) + L1, Tb=Tb, dtype=dtype, top_k=4,
                      ns=1, nr=1, lens=[t + L1 for t in T0])
    refill_k = O.fill_normal(6450 + Tb, 1, 0, (w.B, w.Hkv, L2, w.D), dtype)
    refill_v = O.fill_normal(6450 + Tb, 2, 0, (w.B, w.Hkv, L2, w.D), dtype)
    c = new_cache(w, kv_bits=kv_bits)
    for b in range(w.B):
        c.append(to_dev(np.ascontiguousarray(w.keys[b][None, :, :T0[b]]), dtype, gpu),
                 to_dev(np.ascontiguousarray(w.values[b][None, :, :T0[b]]), dtype, gpu), seq_ids=[b])

    def check(keys, values, T_end, L, q, out, idx):
        got = from_dev(out)
        for b in range(w.B):
            for i in range(L):
                T_i = T_end[b] - L + 1 + i
                for h in range(w.Hkv):
                    ri, ro = _oracle_query(q[b, h * w.G:(h + 1) * w.G, i], keys[b][h], values[b][h], T_i, Tb,
                                           w.ns, w.nr, w.top_k, w.scale, dtype, kv_bits)
                    assert np.array_equal(idx[b, i, h].cpu().numpy(), ri), f"seq {b} query {i} head {h}"
                    err = output_error(O.to_f32(got[b, h * w.G:(h + 1) * w.G, i], dtype).astype(np.float64),
                                       ro, dtype)
                    assert err <= (1e-2 if kv_bits else TOL), f"seq {b} query {i} head {h}: {err:.3g}"
        for b in range(w.B):
            s = from_dev(c.exportSummaries(b))
            for h in range(w.Hkv):
                if kv_bits:
                    ref = O.summaries_q(*O.quantize(np.ascontiguousarray(keys[b][h][:T_end[b]]), kv_bits, 64),
                                       Tb, kv_bits, 64)
                else:
                    ref = O.summaries(np.ascontiguousarray(keys[b][h][:T_end[b]]), Tb, dtype)
                assert np.array_equal(s[h], ref), f"seq {b} head {h}: summaries"

    # the draft pass: 5 tokens, completing a block
    dk = np.stack([k[:, T0[b]:T0[b] + L1] for b, k in enumerate(w.keys)])
    dv = np.stack([v[:, T0[b]:T0[b] + L1] for b, v in enumerate(w.values)])
    c.append(to_dev(dk, dtype, gpu), to_dev(dv, dtype, gpu))
    q1 = O.fill_normal(6460, 0, 0, (w.B, w.Hq, L1, w.D), dtype)
    idx1 = torch.empty((w.B, L1, w.Hkv, c.nselMax), dtype=torch.int32, device=gpu)
    o1 = c.decodeMulti(to_dev(q1, dtype, gpu), w.scale, idx_out=idx1)
    torch.cuda.synchronize()
    check(w.keys, w.values, [t + L1 for t in T0], L1, q1, o1, idx1)
    # reject 4: the completed block is partial again
    assert c.trim(REJ) == REJ and [c.seqLen(b) for b in range(w.B)] == [t + 1 for t in T0]
    # 3 different tokens refill it
    c.append(to_dev(refill_k, dtype, gpu), to_dev(refill_v, dtype, gpu))
    keys = [np.concatenate([w.keys[b][:, :T0[b] + 1], refill_k[b]], axis=1) for b in range(w.B)]
    values = [np.concatenate([w.values[b][:, :T0[b] + 1], refill_v[b]], axis=1) for b in range(w.B)]
    q2 = O.fill_normal(6470, 0, 0, (w.B, w.Hq, L2, w.D), dtype)
    idx2 = torch.empty((w.B, L2, w.Hkv, c.nselMax), dtype=torch.int32, device=gpu)
    o2 = c.decodeMulti(to_dev(q2, dtype, gpu), w.scale, idx_out=idx2)
    torch.cuda.synchronize()
    check(keys, values, [t + 1 + L2 for t in T0], L2, q2, o2, idx2)
