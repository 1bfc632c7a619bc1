"""Graph-capturable decode loop: bsattn_reserve, then [bsattn_append_step,
bsattn_decode] captured once in a HIP graph and replayed per step with new
keys / values / queries copied into its input buffers.  Every replay equals
the eager loop (bsattn_append + bsattn_decode) bit for bit, including the
steps that complete a block (the appended token's block summary is written
on the device); the device-side capacity guard and the host-view rules hold."""
from __future__ import annotations

import numpy as np
import pytest

from common import make_workload, new_cache, to_dev

pytestmark = pytest.mark.gpu


def _prefix(w, gpu, caches):
    for c in caches:
        for b in range(w.B):
            c.append(to_dev(np.ascontiguousarray(w.keys[b][None]), w.dtype, gpu),
                     to_dev(np.ascontiguousarray(w.values[b][None]), w.dtype, gpu), seq_ids=[b])


@pytest.mark.parametrize("dtype,Tb,K", [("bf16", 64, 8), ("f16", 32, 24)])
def test_captured_decode_loop_matches_eager(gpu, dtype, Tb, K):
    import torch
    from bsattn import BsattnError
    STEPS = 70
    lens = [1000, 2 * Tb - 3, 3000, 77]
    w = make_workload(8000 + Tb, B=4, Hq=32, Hkv=8, T=max(lens), Tb=Tb, dtype=dtype, top_k=K, lens=lens,
                      salient_frac=0.01)
    mbps = (max(lens) + STEPS) // Tb + 3
    a, b = new_cache(w, mbps=mbps), new_cache(w, mbps=mbps)
    _prefix(w, gpu, (a, b))
    td = torch.bfloat16 if dtype == "bf16" else torch.float16
    g = torch.Generator(device=gpu)
    g.manual_seed(8100 + Tb)
    K_ = torch.randn(STEPS, 4, 8, 1, 128, device=gpu, generator=g).to(td)
    V_ = torch.randn(STEPS, 4, 8, 1, 128, device=gpu, generator=g).to(td)
    Q_ = torch.randn(STEPS, 4, 32, 1, 128, device=gpu, generator=g).to(td)
    a.reserve(STEPS)
    kbuf, vbuf, qbuf = K_[0].clone(), V_[0].clone(), Q_[0].clone()
    # step 0 eagerly through the device-side path (also the warm-up before capture)
    a.appendStep(kbuf, vbuf)
    out0 = a.decode(qbuf, w.scale)
    b.append(K_[0], V_[0])
    ref0 = b.decode(Q_[0], w.scale)
    torch.cuda.synchronize()
    assert torch.equal(out0.view(torch.int16), ref0.view(torch.int16))
    with pytest.raises(BsattnError):
        a.offset  # the host view is stale until sync
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        a.appendStep(kbuf, vbuf)
        out = a.decode(qbuf, w.scale)
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
    assert [a.seqLen(s) for s in range(4)] == [n + STEPS for n in lens]
    for s in range(4):
        assert torch.equal(a.exportSummaries(s), b.exportSummaries(s))
    ka, va = a.export([0, 1, 2, 3][:1])
    kb, vb = b.export([0])
    assert torch.equal(ka, kb) and torch.equal(va, vb)


def test_append_step_stops_at_the_reservation(gpu):
    import torch
    from bsattn import BsattnError
    Tb = 64
    w = make_workload(8200, B=2, Hq=32, Hkv=8, T=Tb - 2, Tb=Tb, dtype="bf16", top_k=2, lens=[Tb - 2, Tb - 2])
    c = new_cache(w, mbps=8)
    _prefix(w, gpu, (c,))
    c.reserve(2)  # the first page holds 2 more tokens: no new page
    k = torch.zeros((2, 8, 1, 128), dtype=torch.bfloat16, device=gpu)
    for _ in range(5):
        c.appendStep(k, k)
    c.sync()
    assert c.seqLen(0) == Tb and c.seqLen(1) == Tb
    # host-driven calls work again after sync; a quantized cache has no device-side appends
    c.append(k, k)
    assert c.seqLen(0) == Tb + 1
    cq = new_cache(make_workload(8201, B=1, Hq=32, Hkv=8, T=64, Tb=64, dtype="f16", top_k=2), kv_bits=4)
    with pytest.raises(BsattnError):
        cq.appendStep(torch.zeros((1, 8, 1, 128), dtype=torch.float16, device=gpu),
                      torch.zeros((1, 8, 1, 128), dtype=torch.float16, device=gpu))


def test_reserved_surplus_does_not_hide_a_shortage(gpu):
    """A sequence holding pages ahead of its length (bsattn_reserve) needs
    none for its next tokens, and its surplus must not offset what another
    sequence needs: a pool of 4 pages (Tb 64), 192 tokens reserved for
    sequence 0 (3 pages), then 128 tokens appended to sequences 0 and 1.
    Sequence 1 needs 2 pages and 1 is free: BSATTN_ERR_NO_PAGES, with the
    free pages and every length unchanged."""
    import torch
    from bsattn import BsattnError, _lib
    Tb = 64
    w = make_workload(8300, B=2, Hq=32, Hkv=8, T=Tb, Tb=Tb, dtype="bf16", top_k=2, lens=[0, 0])
    c = new_cache(w, mbps=8, num_pages=4)
    c.reserve(3 * Tb, seq_ids=[0])
    assert c.freePages == 1
    k = torch.zeros((2, 8, 2 * Tb, 128), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(BsattnError) as e:
        c.append(k, k, seq_ids=[0, 1])
    assert e.value.code == _lib.ERR_NO_PAGES
    assert c.freePages == 1 and c.seqLen(0) == 0 and c.seqLen(1) == 0
    # within the pool: sequence 0 uses its reserved pages, sequence 1 takes the free one
    k1 = k[:, :, :Tb].contiguous()
    c.append(k1, k1, seq_ids=[0, 1])
    torch.cuda.synchronize()
    assert c.freePages == 0 and c.seqLen(0) == Tb and c.seqLen(1) == Tb
