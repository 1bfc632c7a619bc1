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
