"""Page accounting through the C ABI: the seeded free-list permutation (the
shuffled physical order of the 32-sequence decode loop) hands pages out in the
order a Fisher-Yates restatement predicts, block tables list them in logical
order, and results do not depend on the physical order."""
from __future__ import annotations

import numpy as np
import pytest

from common import fill, from_dev, log, make_workload, new_cache, oracle_decode, output_error, to_dev
import oracle as O

pytestmark = pytest.mark.gpu

MASK = (1 << 64) - 1


def _permuted_free_list(num_pages: int, seed: int):
    """The free list is a stack [P-1, ..., 0] (back handed out first);
    step i swaps the (i+1)-th slot from the back with one of the n - i slots
    at or before it, chosen by hash3(seed, 5, i) mod (n - i)."""
    f = list(range(num_pages - 1, -1, -1))
    n = len(f)
    for i in range(n - 1):
        h = int(O.lib().orc_hash3(seed, 5, i)) & MASK
        a = n - 1 - i
        f[a], f[a - h % (n - i)] = f[a - h % (n - i)], f[a]
    return f


def test_shuffled_pages_follow_the_permutation(gpu):
    w = make_workload(5100, B=3, Hq=8, Hkv=8, T=10 * 64, Tb=64, dtype="f16", top_k=2,
                      lens=[10 * 64, 3 * 64 + 5, 64])
    cache = new_cache(w, num_pages=40)
    assert cache.freePages == 40
    cache.shuffleFreePages(1004)
    f = _permuted_free_list(40, 1004)
    fill(cache, w, gpu)
    want = f[::-1]
    got = [cache.seqPages(b) for b in range(w.B)]
    log(f"[pages] {got}")
    assert got[0] == want[:10]
    assert got[1] == want[10:14]
    assert got[2] == want[14:15]
    assert cache.freePages == 40 - 15
    idx_ref, out_ref = oracle_decode(w)
    q = to_dev(w.q[:, :, None, :], w.dtype, gpu)
    idx = cache.selectBlocks(q).cpu().numpy()
    assert np.array_equal(idx, idx_ref)
    out = from_dev(cache.decode(q, w.scale)).reshape(w.B, w.Hq, w.D)
    assert output_error(O.to_f32(out, w.dtype).astype(np.float64), out_ref, w.dtype) <= 2e-3
    cache.reset([1])
    assert cache.seqPages(1) == []
    assert cache.freePages == 40 - 11
