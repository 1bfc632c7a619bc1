"""bsattn_decode_noalloc (the decode with its workspaces in the library's
fixed per-GPU scratch, nothing allocated) against bsattn_decode, through the
C ABI: selected blocks and outputs bit-identical (same kernels), on two calls
in a row, the second with a smaller batch, for the paths decode takes (fused
decode kernel, selection inside the attention kernel, separate workgroup
selection with MFMA scores); a call whose workspaces exceed the scratch is
refused with BSATTN_ERR_RANGE before any work."""
from __future__ import annotations

import numpy as np
import pytest

from common import fill, log, make_workload, new_cache, oracle_decode, output_error, to_dev
import oracle as O

pytestmark = pytest.mark.gpu


def _both(cache, w, gpu, ids):
    import torch
    q = to_dev(w.q[ids][:, :, None, :], w.dtype, gpu)
    nsel = cache.nselMax
    ia = torch.full((len(ids), w.Hkv, nsel), -7, dtype=torch.int32, device=gpu)
    ib = torch.full_like(ia, -9)
    ref = cache.decode(q, w.scale, seq_ids=ids, idx_out=ia)
    out = torch.full_like(q, 3.0)
    got = cache.decodeNoAlloc(q, w.scale, out, seq_ids=ids, idx_out=ib)
    torch.cuda.synchronize()
    assert torch.equal(ia, ib), "selected blocks differ"
    assert torch.equal(ref.view(torch.int16), got.view(torch.int16)), "outputs differ"
    return got


@pytest.mark.parametrize("Hq,Hkv,T,dtype,K", [
    (32, 8, 64 * 40 + 9, "f16", 8),     # fused decode kernel (few candidates)
    (32, 8, 32768, "bf16", 32),         # selection inside the attention kernel
    (64, 4, 64 * 1100, "f16", 16),      # GQA 16: MFMA scores + workgroup selection
])
def test_noalloc_matches_decode_twice(gpu, Hq, Hkv, T, dtype, K):
    log(f"[noalloc] Hq={Hq} Hkv={Hkv} T={T} {dtype}")
    lens = [T, T - 100, T // 2, 700, T - 1, 3000]
    w = make_workload(9700 + Hq + K, B=len(lens), Hq=Hq, Hkv=Hkv, T=T, Tb=64, dtype=dtype, top_k=K,
                      lens=lens)
    cache = new_cache(w)
    fill(cache, w, gpu)
    got = _both(cache, w, gpu, [0, 1, 2, 3, 4, 5])
    # the oracle agrees as well (both are the decode kernels)
    idx_ref, out_ref = oracle_decode(w)
    from common import from_dev
    err = output_error(O.to_f32(from_dev(got).reshape(w.B, Hq, 128), dtype).astype(np.float64), out_ref, dtype)
    assert err <= 2e-3
    # a second call with a smaller batch (reused scratch, other entries)
    _both(cache, w, gpu, [4, 1])


def test_noalloc_refuses_what_the_scratch_cannot_hold(gpu):
    """64 sequences x 64 q heads x 129 splits of 130 floats need ~275 MB of
    partials, far past the 16 MiB scratch: refused with BSATTN_ERR_RANGE
    before any launch; so is a call of more than 64 sequences."""
    import torch
    from bsattn import BsattnError, _lib
    from bsattn import BlockSparseKVCache
    c = BlockSparseKVCache(max_seqs=64, num_q_heads=64, num_kv_heads=4, block_size=32,
                           dtype=torch.float16, top_k=512, sink_blocks=1, recent_blocks=1,
                           max_blocks_per_seq=600, num_pages=64, device=0)
    q = torch.zeros((64, 64, 1, 128), dtype=torch.float16, device=gpu)
    with pytest.raises(BsattnError) as e:
        c.decodeNoAlloc(q, 0.1, torch.empty_like(q))
    assert e.value.code == _lib.ERR_RANGE and "scratch" in str(e.value)
    c2 = BlockSparseKVCache(max_seqs=80, num_q_heads=32, num_kv_heads=8, block_size=64,
                            dtype=torch.float16, top_k=4, max_blocks_per_seq=4, device=0)
    q65 = torch.zeros((65, 32, 1, 128), dtype=torch.float16, device=gpu)
    with pytest.raises(BsattnError) as e:
        c2.decodeNoAlloc(q65, 0.1, torch.empty_like(q65))
    assert e.value.code == _lib.ERR_RANGE


def test_noalloc_captured_after_append_step(gpu):
    """A captured [appendStep, decodeNoAlloc] step (device-side lengths, no
    bsattn_sync in between), replayed with new inputs copied in, equals the
    eager append + decode bit for bit at every step, across block fills;
    the scratch address is looked up by one call before the capture."""
    import torch
    STEPS, Tb = 40, 64
    lens = [900, 2 * Tb - 3, 2500]
    w = make_workload(9800, B=3, Hq=32, Hkv=8, T=max(lens), Tb=Tb, dtype="bf16", top_k=8, lens=lens,
                      salient_frac=0.01)
    mbps = (max(lens) + STEPS) // Tb + 3
    a, b = new_cache(w, mbps=mbps), new_cache(w, mbps=mbps)
    fill(a, w, gpu)
    fill(b, w, gpu)
    g = torch.Generator(device=gpu)
    g.manual_seed(9801)
    K_ = torch.randn(STEPS, 3, 8, 1, 128, device=gpu, generator=g).to(torch.bfloat16)
    V_ = torch.randn(STEPS, 3, 8, 1, 128, device=gpu, generator=g).to(torch.bfloat16)
    Q_ = torch.randn(STEPS, 3, 32, 1, 128, device=gpu, generator=g).to(torch.bfloat16)
    a.reserve(STEPS)
    kbuf, vbuf, qbuf = K_[0].clone(), V_[0].clone(), Q_[0].clone()
    out = torch.empty_like(qbuf)
    # step 0 eagerly (warms the scratch lookup before the capture)
    a.appendStep(kbuf, vbuf)
    a.decodeNoAlloc(qbuf, w.scale, out)
    b.append(K_[0], V_[0])
    ref = b.decode(Q_[0], w.scale)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), "step 0 differs"
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        a.appendStep(kbuf, vbuf)
        a.decodeNoAlloc(qbuf, w.scale, out)
    for i in range(1, STEPS):
        kbuf.copy_(K_[i])
        vbuf.copy_(V_[i])
        qbuf.copy_(Q_[i])
        gr.replay()
        b.append(K_[i], V_[i])
        ref = b.decode(Q_[i], w.scale)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"step {i} differs"
    a.sync()
    assert [a.seqLen(s) for s in range(3)] == [n + STEPS for n in lens]
